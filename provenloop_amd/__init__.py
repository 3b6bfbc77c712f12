"""MI355X (gfx950) CKKS engine for TenSafe's encrypted LoRA-delta path.

Modules:
  tensafe_he  -- the reference's Python backend interface (CkksContext & co.)
  adapter     -- drop-in for the engine's _TenSafeHEAdapter (Try 0 backend)
  zero_moai   -- column-packed ct x pt LoRA matvec (packing, batching, extraction)
  _lib        -- ctypes binding of the C ABI (include/tensafe_he.h)
"""
__version__ = "0.1.0"
