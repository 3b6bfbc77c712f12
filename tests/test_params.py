"""The library's 8-limb N = 32768 chain follows its stated rule (CPU only)."""
from oracle import oracle as orc
from provenloop_amd.params import CHAIN_N32768_L8


def test_chain_n32768_l8_rule():
    ref = orc.default_chain(32768)
    c = CHAIN_N32768_L8
    assert len(c) == 8 and len(set(c)) == 8
    assert c[:3] == ref[:3] and c[-1] == ref[-1]
    for q in c:
        assert q % 65536 == 1 and q < 2 ** 61
        assert orc.is_prime(q)
    # the inserted limbs are the next four primes = 1 mod 2N below q2, in descending order
    want, q = [], ref[2] - 65536
    while len(want) < 4:
        if orc.is_prime(q):
            want.append(q)
        q -= 65536
    assert c[3:7] == want
    # every candidate skipped between them is composite
    for hi, lo in zip([ref[2]] + want[:-1], want):
        assert not any(orc.is_prime(x) for x in range(lo + 65536, hi, 65536))


def test_oracle_accepts_chain():
    ctx = orc.Context(32768, CHAIN_N32768_L8)
    assert ctx.L == 8 and ctx.moduli == CHAIN_N32768_L8
