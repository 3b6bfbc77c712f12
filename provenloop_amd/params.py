"""Modulus chains beyond the reference's (tensafe-he-core/src/params.rs:66-126).

CHAIN_N32768_L8 is the 8-limb chain of the saturation workload (Qwen2.5-7B
shape, N = 32768, scale 2^40). The reference defines only a 4-limb chain for
N = 32768 (params.rs:109-126) and its `CkksParams::custom` repeats primes
when bit widths repeat (params.rs:142-193), so this chain is the library's
own, built by one rule: the reference's N = 32768 chain
[q0 (60 bit), q1, q2 (40 bit), q3 (60 bit)] with the next four primes
q = 1 mod 2N below q2 inserted before q3. Every prime is distinct and
NTT-friendly for N = 32768 (q = 1 mod 65536); the last prime stays the
60-bit q3, so a rescale leaves scale 2^80 / q3 as it does on the reference
chain.
"""

CHAIN_N32768_L8 = [
    1152921504606584833,  # reference q0 (60 bit)
    1099507695617,        # reference q1 (40 bit)
    1099506515969,        # reference q2 (40 bit)
    1099504549889,        # next primes = 1 mod 65536 below q2
    1099503894529,
    1099503370241,
    1099502714881,
    1152921504598720513,  # reference q3 (60 bit)
]
