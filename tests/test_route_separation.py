"""The rule by which one-token gate/up workgroups take their expert set
from the exps alone (route_set_by_exps, kernels.hip): with e = exp(x - max)
in [0, 1] and inv = 1 / sum in [1/256, 1], two exps e_a > e_b whose f32
bit patterns are at least 16 apart, with e_b >= 2^-100 (or e_b = +0 and
e_a >= 2^-100), give probabilities RN(e_a * inv) > RN(e_b * inv).  Checked
here in IEEE f32 arithmetic (numpy) on random and edge cases; a rule that
were one ulp too loose fails on the tight cases."""
import numpy as np

TINY = np.float32(2.0 ** -100)


def _f(bits):
    return np.asarray(bits, np.uint32).view(np.float32)


def _p(e, inv):
    return (np.asarray(e, np.float32) * np.asarray(inv, np.float32)).astype(np.float32)


def _allowed(ea, eb):
    ba, bb = np.asarray(ea, np.float32).view(np.uint32), np.asarray(eb, np.float32).view(np.uint32)
    sep = (bb.astype(np.int64) + 16 <= ba.astype(np.int64)) & (eb >= TINY)
    return sep | ((eb == 0) & (ea >= TINY))


def test_random_pairs_stay_ordered():
    rng = np.random.default_rng(11)
    n = 2_000_000
    eb = _f(rng.integers(_f_bits(TINY), _f_bits(np.float32(1.0)), n, dtype=np.uint32))
    gap = rng.integers(16, 200, n).astype(np.uint32)
    ea = _f(np.minimum(eb.view(np.uint32) + gap, _f_bits(np.float32(1.0))))
    inv = (1.0 / rng.uniform(1.0, 256.0, n)).astype(np.float32)
    ok = _allowed(ea, eb)
    assert ok.mean() > 0.99
    assert np.all(_p(ea[ok], inv[ok]) > _p(eb[ok], inv[ok]))


def test_tight_cases():
    # 16 ulps apart at the smallest exps allowed and the extreme inverses,
    # across binade edges, and +0 below the smallest allowed exp
    invs = np.array([1.0, 1.0 / 256.0, np.nextafter(np.float32(1.0 / 256.0), np.float32(1.0)),
                     np.float32(0.7), np.float32(1.0 / 3.0)], np.float32)
    base = [TINY, np.float32(2.0 ** -24), np.float32(0.5), np.nextafter(np.float32(0.5), np.float32(0)),
            np.float32(1.0) - np.float32(2.0 ** -24) * 16]
    for eb in base:
        ea = _f(np.float32(eb).view(np.uint32) + 16)
        assert _allowed(ea, eb)
        for inv in invs:
            assert _p(ea, inv) > _p(eb, inv), (eb, inv)
    for inv in invs:
        assert _p(TINY, inv) > _p(np.float32(0.0), inv)


def test_looser_rules_fail():
    # the 16 and the 2^-100 are not slack that can be dropped: equal
    # probabilities appear for pairs the rule refuses
    rng = np.random.default_rng(12)
    n = 2_000_000
    eb = _f(rng.integers(_f_bits(TINY), _f_bits(np.float32(1.0)), n, dtype=np.uint32))
    ea = _f(eb.view(np.uint32) + 1)
    inv = (1.0 / rng.uniform(1.0, 256.0, n)).astype(np.float32)
    assert np.any(_p(ea, inv) == _p(eb, inv))
    tiny_b = _f(rng.integers(1, _f_bits(TINY), n, dtype=np.uint32))
    tiny_a = _f(tiny_b.view(np.uint32) + 16)
    assert np.any(_p(tiny_a, np.float32(1.0 / 256.0)) == _p(tiny_b, np.float32(1.0 / 256.0)))


def _f_bits(x):
    return int(np.float32(x).view(np.uint32))
