"""CPU: pin the oracle (oracle/attention_oracle.py).

Each check is chosen so that a plausible mistake in the oracle (a dropped
scale, the mask shifted by one, a transposed operand, a missing max
subtraction, the LSE in base 2) fails at least one of them; the mutant tests at
the end plant exactly those mistakes in copies of the oracle and assert that
the pins reject them.
"""

from __future__ import annotations

import math

import numpy as np
import pytest
import scipy.special

from oracle.attention_oracle import (
    attention_bruteforce,
    attention_flops,
    attention_ref,
    round_bf16,
    round_fp16,
)

RNG = np.random.default_rng(20261201)


def rand(*shape, scale=1.0):
    return (RNG.standard_normal(shape) * scale).astype(np.float32)


# ---------------------------------------------------------------------------
# Pins, written against a generic oracle `fn(q, k, v, causal, scale) -> (o, lse)`.

def pin_bruteforce(fn, tol=2e-5):
    for sq, d, causal in [(1, 8, False), (5, 8, True), (17, 16, False), (17, 16, True), (37, 64, True)]:
        q, k, v = rand(sq, d), rand(sq, d), rand(sq, d)
        o, lse = fn(q, k, v, causal, 0.37)
        ob, lb = attention_bruteforce(q, k, v, causal, 0.37)
        if not (np.abs(o - ob).max() <= tol and np.abs(lse - lb).max() <= tol):
            return False
    # Sq != Sk non-causal (rectangular)
    q, k, v = rand(3, 8), rand(11, 8), rand(11, 8)
    o, lse = fn(q, k, v, False, 0.5)
    ob, lb = attention_bruteforce(q, k, v, False, 0.5)
    return np.abs(o - ob).max() <= tol and np.abs(lse - lb).max() <= tol


def pin_zero_keys(fn):
    """K = 0: every visible logit is 0, so weights are uniform.

    Non-causal: O = mean(V), LSE = ln(Sk).  Causal row i: O_i = mean(V[:i+1]),
    LSE_i = ln(i + 1).
    """
    s, d = 23, 16
    q, k, v = rand(s, d), np.zeros((s, d), np.float32), rand(s, d)
    o, lse = fn(q, k, v, False, 0.9)
    ok = np.allclose(o, np.broadcast_to(v.mean(0), o.shape), atol=1e-5)
    ok &= np.allclose(lse, math.log(s), atol=1e-5)
    o, lse = fn(q, k, v, True, 0.9)
    want = np.cumsum(v, 0) / np.arange(1, s + 1)[:, None]
    ok &= np.allclose(o, want, atol=1e-5)
    ok &= np.allclose(lse, np.log(np.arange(1, s + 1)), atol=1e-5)
    return bool(ok)


def pin_first_causal_row(fn):
    """Causal row 0 sees only key 0: O_0 = V_0 and LSE_0 = scale * q_0 . k_0."""
    q, k, v = rand(9, 32), rand(9, 32), rand(9, 32)
    o, lse = fn(q, k, v, True, 0.21)
    return bool(np.allclose(o[0], v[0], atol=1e-6) and abs(lse[0] - 0.21 * float(q[0] @ k[0])) <= 1e-5)


def pin_shift(fn):
    """Adding c to every logit leaves O unchanged and raises LSE by c.

    The shift is built into the operands: q' = [q, 1], k' = [k, c / scale].
    """
    s, d, scale, c = 19, 16, 0.3, 2.5
    q, k, v = rand(s, d), rand(s, d), rand(s, d)
    q2 = np.concatenate([q, np.ones((s, 1), np.float32)], 1)
    k2 = np.concatenate([k, np.full((s, 1), c / scale, np.float32)], 1)
    ok = True
    for causal in (False, True):
        o1, l1 = fn(q, k, v, causal, scale)
        o2, l2 = fn(q2, k2, v, causal, scale)
        ok &= np.allclose(o1, o2, atol=1e-5) and np.allclose(l2 - l1, c, atol=1e-4)
    return bool(ok)


def pin_one_hot(fn):
    """One-hot q_i = e_{p(i)}, k_j = e_j with a large scale: row i selects V[p(i)]."""
    s = 12
    perm = RNG.permutation(s)
    q = np.eye(s, dtype=np.float32)[perm]
    k = np.eye(s, dtype=np.float32)
    v = rand(s, 8)
    o, lse = fn(q, k, v, False, 60.0)
    return bool(np.allclose(o, v[perm], atol=1e-5) and np.allclose(lse, 60.0, atol=1e-4))


def pin_causal_prefix(fn):
    """Causal row i equals non-causal attention of q_i over keys [0, i]."""
    s, d = 14, 16
    q, k, v = rand(s, d), rand(s, d), rand(s, d)
    o, lse = fn(q, k, v, True, 0.4)
    for i in (0, 3, 9, 13):
        oi, li = fn(q[i:i + 1], k[:i + 1], v[:i + 1], False, 0.4)
        if not (np.allclose(o[i], oi[0], atol=1e-6) and abs(lse[i] - li[0]) <= 1e-6):
            return False
    return True


def pin_library(fn):
    """scipy.special.softmax / logsumexp (an independent implementation) on the logits."""
    s, d = 31, 64
    q, k, v = rand(s, d), rand(s, d), rand(s, d)
    logits = (q.astype(np.float64) @ k.astype(np.float64).T) * 0.125
    logits[np.triu_indices(s, 1)] = -np.inf
    o, lse = fn(q, k, v, True, 0.125)
    want_o = scipy.special.softmax(logits, axis=-1) @ v.astype(np.float64)
    want_l = scipy.special.logsumexp(logits, axis=-1)
    return bool(np.allclose(o, want_o, atol=2e-5) and np.allclose(lse, want_l, atol=2e-5))


def pin_large_logits(fn):
    """Logits far beyond exp's range (|s| ~ 1e3): the max-subtraction must keep it finite."""
    s, d = 16, 8
    q, k, v = rand(s, d) * 30, rand(s, d) * 30, rand(s, d)
    o, lse = fn(q, k, v, False, 1.0)
    ob, lb = attention_bruteforce(q, k, v, False, 1.0)
    return bool(np.isfinite(o).all() and np.allclose(o, ob, atol=1e-4) and np.allclose(lse, lb, rtol=1e-6))


PINS = [pin_bruteforce, pin_zero_keys, pin_first_causal_row, pin_shift, pin_one_hot,
        pin_causal_prefix, pin_library, pin_large_logits]


def oracle(q, k, v, causal, scale):
    return attention_ref(q, k, v, causal, scale)


@pytest.mark.parametrize("pin", PINS, ids=[p.__name__ for p in PINS])
def test_oracle_pins(pin):
    assert pin(oracle)


# ---------------------------------------------------------------------------
# Mutants: each plants one plausible mistake; at least one pin must reject it.

def _mutant_no_scale(q, k, v, causal, scale):
    return attention_ref(q, k, v, causal, 1.0)


def _mutant_mask_off_by_one(q, k, v, causal, scale):
    # Masks the diagonal as well (triu with k=0): row 0 would see no key at all,
    # so emulate "j < i" visibility plus key 0 for row 0.
    q = np.asarray(q, np.float32)
    o, lse = attention_ref(q, k, v, False, scale)
    if not causal:
        return o, lse
    s = q.shape[0]
    out = np.empty_like(o)
    lo = np.empty_like(lse)
    for i in range(s):
        hi = max(i, 1)
        oi, li = attention_ref(q[i:i + 1], k[:hi], v[:hi], False, scale)
        out[i], lo[i] = oi[0], li[0]
    return out, lo


def _mutant_transposed_scores(q, k, v, causal, scale):
    # Uses K Q^T instead of Q K^T (scores transposed) before the softmax.
    q = np.asarray(q, np.float32)
    k = np.asarray(k, np.float32)
    if q.shape[0] != k.shape[0]:
        return attention_ref(q, k, v, causal, scale)
    s = (k @ q.T) * scale
    if causal:
        s = np.where(np.triu(np.ones_like(s, bool), 1), -np.inf, s)
    m = s.max(-1, keepdims=True)
    e = np.exp(s - m)
    return (e / e.sum(-1, keepdims=True)) @ v, (np.log(e.sum(-1)) + m[:, 0]).astype(np.float32)


def _mutant_lse_base2(q, k, v, causal, scale):
    o, lse = attention_ref(q, k, v, causal, scale)
    return o, lse / np.float32(math.log(2.0))


def _mutant_unstable(q, k, v, causal, scale):
    # No max subtraction (the reference's "lazy" path, flash_attention_forward.py:725-752).
    q = np.asarray(q, np.float32)
    s = (q @ np.asarray(k, np.float32).T) * np.float32(scale)
    if causal:
        s = np.where(np.triu(np.ones_like(s, bool), 1), -np.inf, s)
    with np.errstate(over="ignore", invalid="ignore"):
        e = np.exp(s)
        return (e / e.sum(-1, keepdims=True)) @ v, np.log(e.sum(-1)).astype(np.float32)


MUTANTS = [_mutant_no_scale, _mutant_mask_off_by_one, _mutant_transposed_scores,
           _mutant_lse_base2, _mutant_unstable]


@pytest.mark.parametrize("mutant", MUTANTS, ids=[m.__name__ for m in MUTANTS])
def test_pins_reject_mutant(mutant):
    with np.errstate(all="ignore"):
        results = [pin(mutant) for pin in PINS]
    assert not all(results), f"{mutant.__name__} passed every pin"


# ---------------------------------------------------------------------------
# Rounding helpers and shape handling.

def test_round_bf16_matches_torch():
    torch = pytest.importorskip("torch")
    x = np.concatenate([rand(4096) * 10, np.array([0.0, -0.0, 1.0, 1.00390625, 1.005859375, 3.0e38,
                                                   -3.0e38, 1e-40, np.inf, -np.inf], np.float32)])
    want = torch.from_numpy(x).to(torch.bfloat16).float().numpy()
    np.testing.assert_array_equal(round_bf16(x), want)
    assert np.isnan(round_bf16(np.array([np.nan], np.float32)))[0]


def test_round_fp16_matches_torch():
    torch = pytest.importorskip("torch")
    x = rand(4096) * 100
    want = torch.from_numpy(x).to(torch.float16).float().numpy()
    np.testing.assert_array_equal(round_fp16(x), want)


def test_batched_shapes_and_rounding():
    q, k, v = rand(2, 3, 20, 16), rand(2, 3, 20, 16), rand(2, 3, 20, 16)
    o, lse = attention_ref(q, k, v, True, 0.25, out_dtype="bfloat16")
    assert o.shape == (2, 3, 20, 16) and lse.shape == (2, 3, 20)
    o1, l1 = attention_ref(q[1, 2], k[1, 2], v[1, 2], True, 0.25)
    np.testing.assert_array_equal(o[1, 2], round_bf16(o1))
    np.testing.assert_allclose(lse[1, 2], l1, atol=1e-6)


def test_flops_formula():
    assert attention_flops(4, 32, 2048, 2048, 128, True) == pytest.approx(1.3744e11, rel=1e-4)
    assert attention_flops(1, 8, 512, 512, 64, False) == pytest.approx(5.369e8, rel=1e-3)


def test_rejects_mismatched_shapes():
    with pytest.raises(ValueError):
        attention_ref(rand(4, 8), rand(4, 16), rand(4, 16), False, 1.0)
    with pytest.raises(ValueError):
        attention_ref(rand(2, 4, 8), rand(3, 4, 8), rand(3, 4, 8), False, 1.0)


# ---------------------------------------------------------------------------
# Split-KV restatement: partial attention over key ranges + LSE merge.

from oracle.attention_oracle import attention_partial, merge_partials  # noqa: E402


def _partition_check(merge, partial=attention_partial, seed=5, sq=37, sk=37, d=16, causal=True,
                     cuts=(0, 5, 16, 30, 37), scale=0.3):
    rng = np.random.default_rng(seed)
    q = rng.standard_normal((2, sq, d)).astype(np.float32)
    k = rng.standard_normal((2, sk, d)).astype(np.float32)
    v = rng.standard_normal((2, sk, d)).astype(np.float32)
    want_o, want_l = attention_ref(q, k, v, causal, scale)
    parts = [partial(q, k, v, causal, scale, lo, hi) for lo, hi in zip(cuts[:-1], cuts[1:])]
    with np.errstate(over="ignore", invalid="ignore"):
        got_o, got_l = merge(parts)
    return float(np.nan_to_num(np.abs(got_o - want_o), nan=np.inf).max()), \
        float(np.nan_to_num(np.abs(got_l - want_l), nan=np.inf).max())


@pytest.mark.parametrize("causal", [False, True])
@pytest.mark.parametrize("cuts", [(0, 37), (0, 5, 16, 30, 37), (0, 1, 2, 3, 37), (0, 36, 37), (0, 12, 24, 48)])
@pytest.mark.parametrize("scale", [0.3, 40.0])
def test_merge_of_partials_is_full_attention(causal, cuts, scale):
    """Any partition of the keys (empty and single-key runs, runs past Sk) merges back exactly,
    also with logits large enough that exp(LSE) overflows float32 (scale 40)."""
    d_o, d_l = _partition_check(merge_partials, causal=causal, cuts=cuts, scale=scale)
    assert d_o < 1e-5 and d_l < 2e-6 * max(1.0, scale)  # float32 rounding of both sides


def test_partial_matches_bruteforce_on_a_range():
    rng = np.random.default_rng(9)
    q, k, v = (rng.standard_normal((9, 8)).astype(np.float32) for _ in range(3))
    o, l = attention_partial(q, k, v, True, 0.5, 3, 7)
    for i in range(9):
        keys = [j for j in range(3, 7) if j <= i]
        if not keys:
            assert l[i] == -np.inf and not o[i].any()
            continue
        s = np.array([0.5 * float(q[i] @ k[j]) for j in keys], dtype=np.float64)
        lse = s.max() + math.log(np.exp(s - s.max()).sum())
        want = sum(math.exp(sj - lse) * v[j].astype(np.float64) for sj, j in zip(s, keys))
        assert abs(l[i] - lse) < 1e-5 and np.abs(o[i] - want).max() < 1e-5


def _merge_mutant_unweighted(parts):   # plain average of the partial outputs
    o = np.mean([p[0] for p in parts], axis=0)
    return o.astype(np.float32), merge_partials(parts)[1]


def _merge_mutant_no_max(parts):       # weights exp(LSE_s) without the max shift: overflows in float32
    lses = np.stack([p[1] for p in parts]).astype(np.float32)
    w = np.exp(lses)
    lse = np.log(w.sum(axis=0))
    o = (w[..., None] * np.stack([p[0] for p in parts])).sum(axis=0) / w.sum(axis=0)[..., None]
    return o.astype(np.float32), lse.astype(np.float32)


def _merge_mutant_base2(parts):        # weights in base 2
    lses = np.stack([p[1] for p in parts]).astype(np.float64)
    m = lses.max(axis=0)
    w = np.where(np.isfinite(lses), np.exp2(lses - m), 0.0)
    o = (w[..., None] * np.stack([p[0] for p in parts])).sum(axis=0) / w.sum(axis=0)[..., None]
    return o.astype(np.float32), (m + np.log(w.sum(axis=0))).astype(np.float32)


@pytest.mark.parametrize("mutant", [_merge_mutant_unweighted, _merge_mutant_no_max, _merge_mutant_base2],
                         ids=["unweighted", "no_max", "base2"])
def test_partition_identity_rejects_merge_mutants(mutant):
    results = [_partition_check(mutant, causal=True, cuts=(0, 5, 16, 30, 37), scale=sc) for sc in (0.3, 40.0)]
    assert any(d_o > 1e-3 or d_l > 1e-3 for d_o, d_l in results)


# ---------------------------------------------------------------------------
# fp8-e5m2 V (reference flash_attention_forward.py:704, :737, :996)

from oracle.attention_oracle import attention_fp8v, round_e5m2  # noqa: E402

# (x, e5m2(x)) from the format: binade [2^e, 2^(e+1)) spaced 2^(e-2) for
# e >= -14, subnormals spaced 2^-16, ties to the even mantissa, overflow to inf.
E5M2_KAT = [
    (1.0, 1.0), (1.125, 1.0), (1.1875, 1.25), (1.375, 1.5), (1.625, 1.5), (1.875, 2.0),
    (-1.375, -1.5), (3.0, 3.0), (0.1, 0.09375), (57344.0, 57344.0), (60000.0, 57344.0),
    (61439.0, 57344.0), (61440.0, math.inf), (1e9, math.inf), (-61440.0, -math.inf),
    (2.0 ** -14, 2.0 ** -14), (1.5 * 2.0 ** -16, 2.0 ** -15), (2.0 ** -17, 0.0),
    (0.75 * 2.0 ** -16, 2.0 ** -16), (1.25 * 2.0 ** -16, 2.0 ** -16), (0.0, 0.0),
]


def _e5m2_kat_holds(fn):
    x = np.array([a for a, _ in E5M2_KAT], dtype=np.float32)
    want = np.array([b for _, b in E5M2_KAT], dtype=np.float32)
    return bool(np.array_equal(fn(x), want))


def test_round_e5m2_known_values():
    assert _e5m2_kat_holds(round_e5m2)


def _e5m2_truncating(x):
    x = np.asarray(x, dtype=np.float32)
    ax = np.abs(x).astype(np.float64)
    _, ex = np.frexp(np.where(ax > 0, ax, 1.0))
    q = np.exp2(np.maximum(ex - 1.0, -14.0) - 2.0)
    return np.copysign(np.floor(ax / q) * q, x).astype(np.float32)


def _e5m2_no_subnormals(x):
    r = round_e5m2(x)
    return np.where(np.abs(r) < 2.0 ** -14, np.float32(0), r)


@pytest.mark.parametrize("mutant", [_e5m2_truncating, _e5m2_no_subnormals])
def test_e5m2_kat_rejects_mutants(mutant):
    assert not _e5m2_kat_holds(mutant)


def test_round_e5m2_matches_torch():
    torch = pytest.importorskip("torch")
    rs = np.random.RandomState(3)
    x = np.concatenate([rs.standard_normal(100_000).astype(np.float32) * s
                        for s in (1e-6, 1e-4, 1e-2, 1.0, 1e2, 1e4)]
                       + [np.array([a for a, _ in E5M2_KAT], dtype=np.float32)])
    want = torch.from_numpy(x).to(torch.float8_e5m2).float().numpy()
    assert np.array_equal(round_e5m2(x), want)


def _qkv(rs, shape):
    q = rs.standard_normal(shape).astype(np.float32)
    k = rs.standard_normal(shape).astype(np.float32)
    v = round_e5m2(rs.standard_normal(shape).astype(np.float32))
    return q, k, v


@pytest.mark.parametrize("causal", [False, True])
@pytest.mark.parametrize("block_n,thr", [(64, 8.0), (16, 0.0), (7, 3.0)])
def test_fp8v_replay_without_cast_is_attention(causal, block_n, thr):
    # Online softmax over any tiling and any lazy threshold equals softmax.
    rs = np.random.RandomState(4)
    q, k, v = _qkv(rs, (2, 70, 64))
    o, l = attention_fp8v(q, k, v, causal, 0.125, block_n=block_n, lazy_threshold=thr, round_p=False)
    o_ref, l_ref = attention_ref(q, k, v, causal, 0.125)
    assert np.abs(o - o_ref).max() < 2e-6 and np.abs(l - l_ref).max() < 2e-6


def _jump_inputs(rs, shape, row, key, jump):
    # q row `row` and k row `key` aligned so their logit exceeds every earlier
    # one by about `jump` log2 units at sm_scale 0.125.
    q, k, v = _qkv(rs, shape)
    d = shape[-1]
    u = np.ones(d, dtype=np.float32) / np.sqrt(d)
    q[..., row, :] = u * 8.0
    k[..., key, :] = u * np.float32(jump / (8.0 * 0.125 * 1.4426950408889634))
    return q, k, v


@pytest.mark.parametrize("causal", [False, True])
@pytest.mark.parametrize("bound", [16384.0, 1.0, 1e-3])
def test_fp8v_sum_schedule_without_cast_is_attention(causal, bound):
    # The sum schedule (first tile's max, moves per 32-row group past a lane
    # sum bound) is an online softmax too: without the cast it is softmax,
    # also when a logit jump (row 40, key 150) moves the max and when the
    # bound forces moves on most tiles.
    rs = np.random.RandomState(14)
    q, k, v = _jump_inputs(rs, (2, 200, 64), 40, 150, 30.0)
    o, l = attention_fp8v(q, k, v, causal, 0.125, round_p=False, schedule="sum", sum_bound=bound)
    o_ref, l_ref = attention_ref(q, k, v, causal, 0.125)
    # A few fp32 ulps (row 40's LSE is ~21).
    assert np.abs(o - o_ref).max() < 2e-6
    assert np.all(np.abs(l - l_ref) <= 1e-6 * (1.0 + np.abs(l_ref)))


def test_fp8v_sum_schedule_moves_per_group():
    # A logit 30 log2 units past row 40's first-tile max (key 150) gives
    # p ~ 2^30, past e5m2's range: the sum schedule moves m for row 40's
    # group (rows 32..63) and stays within the e5m2 bound of attention; a
    # schedule that never moves (bound = inf) overflows there.  Rows of other
    # groups keep their max and match the never-move replay bit for bit.
    rs = np.random.RandomState(15)
    q, k, v = _jump_inputs(rs, (1, 200, 64), 40, 150, 30.0)
    o, l = attention_fp8v(q, k, v, False, 0.125, schedule="sum")
    o_ref, l_ref = attention_ref(q, k, v, False, 0.125)
    bound = 2.0 ** -3 * (_probs(q, k, False, 0.125) @ np.abs(v).astype(np.float64)) + 1e-6
    assert np.all(np.abs(o - o_ref) <= bound)
    assert np.all(np.abs(l - l_ref) <= 1e-6 * (1.0 + np.abs(l_ref)))
    with np.errstate(all="ignore"):
        o_never, _ = attention_fp8v(q, k, v, False, 0.125, schedule="sum", sum_bound=np.inf)
    assert not np.isfinite(o_never[0, 40]).all()
    others = np.r_[0:32, 64:200]
    assert np.array_equal(o[0, others], o_never[0, others])


def _probs(q, k, causal, scale):
    s = (q.astype(np.float64) @ k.astype(np.float64).swapaxes(-1, -2)) * scale
    if causal:
        s = np.where(np.triu(np.ones(s.shape[-2:], dtype=bool), k=1), -np.inf, s)
    s = s - s.max(axis=-1, keepdims=True)
    e = np.exp(s)
    return e / e.sum(axis=-1, keepdims=True)


@pytest.mark.parametrize("schedule", ["max", "sum"])
@pytest.mark.parametrize("causal", [False, True])
def test_fp8v_within_e5m2_bound_of_attention(causal, schedule):
    # Rounding each p to nearest e5m2 moves it by at most 2^-3 p, so
    # |O - O_ref| <= 2^-3 sum_j (p_j / l) |v_j| elementwise; l (and LSE) use
    # the unrounded p.
    rs = np.random.RandomState(5)
    q, k, v = _qkv(rs, (2, 150, 64))
    o, l = attention_fp8v(q, k, v, causal, 0.3, schedule=schedule)
    o_ref, l_ref = attention_ref(q, k, v, causal, 0.3)
    bound = 2.0 ** -3 * (_probs(q, k, causal, 0.3) @ np.abs(v).astype(np.float64)) + 1e-6
    assert np.all(np.abs(o - o_ref) <= bound)
    assert np.abs(o - o_ref).max() > 1e-4  # the cast is really applied
    assert np.abs(l - l_ref).max() < 1e-5  # a few fp32 ulps at |LSE| ~ 8


def test_fp8v_single_tile_closed_form():
    # One tile with the exact row max: O = sum_j e5m2(2^(s_j c - m)) v_j / sum_j 2^(s_j c - m).
    rs = np.random.RandomState(6)
    q, k, v = _qkv(rs, (1, 40, 32))
    o, _ = attention_fp8v(q, k, v, False, 0.25, block_n=40, lazy_threshold=0.0)
    c = np.float32(np.float32(0.25) * np.float32(1.4426950408889634))
    s = (q[0].astype(np.float64) @ k[0].astype(np.float64).T).astype(np.float32)
    m = (s.max(axis=1) * c).astype(np.float32)
    p = np.exp2((s.astype(np.float64) * np.float64(c) - m[:, None]).astype(np.float32)).astype(np.float32)
    want = (round_e5m2(p).astype(np.float64) @ v[0]) / p.sum(axis=1, dtype=np.float32)[:, None]
    assert np.abs(o[0] - want).max() < 1e-5
