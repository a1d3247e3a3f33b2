"""CPU oracle for the FlashAttention forward path.

TEST INFRASTRUCTURE ONLY.  Only tests/, __graft_entry__.smoke() and bench.py's
cpu_baseline leg may import this module, and only as the reference that results
are compared against (or the timed CPU baseline).  The product path (flash_attn_npu_amd) never calls it: on a
machine without the HIP library the product raises instead of falling back.

What it restates
----------------
`attention_ref` is the reference's fp32 formula `_torch_attention_reference`
(evaluate_attention.py:134-143), written against numpy instead of torch:

    scores = (q.float() @ k.float()^T) * sm_scale            (:135)
    causal: scores[i, j] = -inf for j > i  (triu(ones, diagonal=1))   (:136-141)
    probs  = softmax(scores, dim=-1) in fp32                 (:142)
    out    = (probs @ v.float()).to(q.dtype)                 (:143)

and adds the natural-log row LSE that the reference kernel stores next to O
(`m_i += log(l_i)`, flash_attention_forward.py:1022, stored fp32 [Z,H,N] at
:1031, allocated at :1136): lse[i] = log(sum_j exp(scores[i, j])) over the
visible keys, i.e. over the *scaled* logits.  The causal convention is the
reference's mask `offs_m >= curr_n` (flash_attention_forward.py:694-696):
key j is visible to query i iff j <= i.

`attention_bruteforce` recomputes the same quantities one row at a time in
float64 with math.exp (a different algorithm: explicit loops, no BLAS); it is
used on tiny inputs to pin `attention_ref`.

`attention_partial` / `merge_partials` restate the split-KV path, which has no
counterpart in the reference: attention over a key range [lo, hi) only (O
normalised by that range's own row sum, LSE over that range, -inf and O = 0
for rows that see no key there), and the exact LSE-weighted merge
    LSE = m + log sum_s exp(LSE_s - m),  O = sum_s exp(LSE_s - LSE) O_s,
with m = max_s LSE_s.  They are pinned by the partition identity: merging the
partials of any partition of the keys reproduces attention_ref
(tests/test_oracle.py, including mutants of the merge).

`attention_fp8v` restates the reference's fp8-e5m2 V path
(flash_attention_forward.py:704, :737, :996): when V is float8e5, the
unnormalised probabilities of each KV tile, p = exp(s - m) against the running
row max m, are cast to e5m2 (`p.to(tl.float8e5)`) before `tl.dot(p, v)`,
while the row sum l accumulates the unrounded fp32 p.  Where the cast falls
depends on the tile size and on when m moves, so the function replays one
schedule, given by `block_n` and `schedule`: tiles of block_n keys from key 0,
exp2 of (s * c - m) with c = |sm_scale| * log2(e) in fp32, and m moved
 * schedule="max": only when a tile's max exceeds it by more than
   lazy_threshold (in log2 units; 0 is the reference's always-move rule);
 * schedule="sum": to the first tile's exact row max, then only for the
   32-row groups (one wavefront's rows) in which some row's sum of p over
   the keys of one half of the tile (keys whose offset in the tile has bit 2
   equal to 0, or to 1) exceeds sum_bound; every row of such a group then
   takes max(m, tile max), O and l are rescaled and p is recomputed.
`round_e5m2` is the OCP e5m2 format
(1 sign, 5 exponent bits with bias 15, 2 mantissa bits, subnormals in steps
of 2^-16, no saturation) with round-to-nearest-even.  Pinning: round_e5m2
against known values from the format definition and against torch's
float8_e5m2 cast; attention_fp8v with the cast disabled against
attention_ref (online softmax = softmax, any block_n / threshold / bound,
including logit jumps that move m under either schedule); with the cast,
against attention_ref within the e5m2 error bound
|O - O_ref| <= 2^-3 * sum_j (p_j / l) |v_j|, and an unchanged LSE; the sum
schedule's move against a never-move mutant (p past e5m2's range).

Rounding helpers produce the fp16 / bf16 values the GPU path writes, so that
an output can be compared to the oracle after the same final cast the
reference applies (`.to(q.dtype)`, evaluate_attention.py:143).

Pinning status: attention_ref and the LSE are pinned by the brute-force loops,
closed forms (zero logits, first causal row, one-hot selection), shift
invariance, the causal-prefix identity and scipy's logsumexp/softmax
(tests/test_oracle.py).  The reference itself cannot execute here (it needs
torch_npu and an Ascend NPU), so there is no reference-produced tensor to
compare against; its only numeric artefact, the accuracy envelope in
evaluation_reports/evaluation_report.txt:10-36, is not a tensor.
"""

from __future__ import annotations

import math

import numpy as np

__all__ = [
    "attention_ref",
    "attention_bruteforce",
    "attention_partial",
    "merge_partials",
    "round_bf16",
    "round_fp16",
    "round_to",
    "round_e5m2",
    "attention_fp8v",
    "attention_flops",
]

LOG2E = 1.4426950408889634
LN2 = 0.6931471805599453


def round_bf16(x: np.ndarray) -> np.ndarray:
    """float32 -> nearest bfloat16 (round to nearest even), returned as float32."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    u = x.view(np.uint32).astype(np.uint64)
    rounded = (u + 0x7FFF + ((u >> 16) & 1)) & 0xFFFF0000
    out = rounded.astype(np.uint32).view(np.float32)
    # NaN must stay NaN (the add above could carry a NaN payload into Inf).
    return np.where(np.isnan(x), np.float32(np.nan), out)


def round_fp16(x: np.ndarray) -> np.ndarray:
    """float32 -> nearest IEEE half (round to nearest even), returned as float32."""
    return np.asarray(x, dtype=np.float32).astype(np.float16).astype(np.float32)


def round_to(x: np.ndarray, dtype: str | None) -> np.ndarray:
    """Apply the final `.to(q.dtype)` of evaluate_attention.py:143."""
    if dtype is None or dtype in ("float32", "fp32"):
        return np.asarray(x, dtype=np.float32)
    if dtype in ("bfloat16", "bf16"):
        return round_bf16(x)
    if dtype in ("float16", "fp16"):
        return round_fp16(x)
    raise ValueError(f"unsupported dtype {dtype!r}")


def round_e5m2(x: np.ndarray) -> np.ndarray:
    """float32 -> nearest OCP fp8-e5m2 value, returned as float32.

    In the binade [2^e, 2^(e+1)) with e >= -14 the e5m2 values are spaced
    2^(e-2); below 2^-14 (subnormals) they are spaced 2^-16.  Ties go to the
    even neighbour; magnitudes that round to 2^16 or beyond (from 61440 =
    (57344 + 65536) / 2 up) become inf, as the cast does without saturation.
    """
    x = np.asarray(x, dtype=np.float32)
    ax = np.abs(x).astype(np.float64)
    finite = np.isfinite(ax)
    _, ex = np.frexp(np.where(finite & (ax > 0), ax, 1.0))  # ax = m 2^ex, m in [0.5, 1)
    e = np.maximum(ex.astype(np.float64) - 1.0, -14.0)
    quantum = np.exp2(e - 2.0)
    r = np.rint(np.where(finite, ax, 0.0) / quantum) * quantum  # rint: half to even
    r = np.where(r >= 65536.0, np.inf, r)
    out = np.copysign(r, x.astype(np.float64)).astype(np.float32)
    return np.where(finite, out, x)


def attention_fp8v(q, k, v8, causal: bool, sm_scale: float, out_dtype: str | None = None,
                   block_n: int = 64, lazy_threshold: float = 8.0, round_p: bool = True,
                   schedule: str = "max", sum_bound: float = 16384.0, group_rows: int = 32):
    """fp8-e5m2 V attention, replaying a tiled online-softmax schedule.

    q, k: [..., S, D] float32 values of the fp16/bf16 inputs; v8: [..., Sk, D]
    float32 values of the e5m2 V.  For each tile of block_n keys (from key 0),
    with m_cand = fp32(max(s) * c) and p = 2^(s * c - m) in fp32 (m taken as
    0 while no key was seen):
      schedule="max": the row max moves to m_cand only when
        m_cand > m + lazy_threshold (O and l are then rescaled by 2^(m - m_new));
      schedule="sum": tile 0 sets m = m_cand; on later tiles p is formed with
        m as it stands, and in every group of group_rows rows where some row's
        sum of p over either half of the tile's keys (offset bit 2 clear / set)
        is not <= sum_bound, each row takes m_new = max(m, m_cand), O and l
        are rescaled by 2^(m - m_new) (1 where m is unchanged) and p is
        recomputed;
    then l += sum(p); O += e5m2(p) @ v  (round_p=False skips the cast).
    Returns (out rounded to out_dtype, lse) like attention_ref.
    """
    if schedule not in ("max", "sum"):
        raise ValueError(f"unknown schedule {schedule!r}")
    q = np.asarray(q, dtype=np.float32)
    k = np.asarray(k, dtype=np.float32)
    v8 = np.asarray(v8, dtype=np.float32)
    lead = q.shape[:-2]
    sq, d = q.shape[-2:]
    sk = k.shape[-2]
    qf = q.reshape(-1, sq, d)
    kf = k.reshape(-1, sk, d)
    vf = v8.reshape(-1, sk, v8.shape[-1]).astype(np.float64)
    c = np.float32(np.float32(abs(sm_scale)) * np.float32(LOG2E))
    thr = np.float32(lazy_threshold)
    bound = np.float32(sum_bound)
    group = np.arange(sq) // group_rows

    def exps(st, m):
        mb = np.where(m == -np.inf, np.float32(0.0), m)
        x = (st.astype(np.float64) * np.float64(c) - mb[:, None].astype(np.float64)).astype(np.float32)
        return np.exp2(x).astype(np.float32)
    out = np.empty((qf.shape[0], sq, vf.shape[-1]), dtype=np.float32)
    lse = np.empty((qf.shape[0], sq), dtype=np.float32)
    rows = np.arange(sq)[:, None]
    for i in range(qf.shape[0]):
        qi = qf[i] if sm_scale >= 0 else -qf[i]
        s_all = (qi.astype(np.float64) @ kf[i].astype(np.float64).T).astype(np.float32)
        m = np.full(sq, -np.inf, dtype=np.float32)
        l = np.zeros(sq, dtype=np.float32)
        acc = np.zeros((sq, vf.shape[-1]), dtype=np.float64)
        for lo in range(0, sk, block_n):
            hi = min(lo + block_n, sk)
            st = s_all[:, lo:hi]
            if causal:
                st = np.where(np.arange(lo, hi)[None, :] > rows, np.float32(-np.inf), st)
            m_cand = (st.max(axis=1) * c).astype(np.float32)
            if schedule == "sum" and lo == 0:
                m = m_cand
                p = exps(st, m)
            elif schedule == "sum":
                p = exps(st, m)
                half = ((np.arange(hi - lo) >> 2) & 1).astype(bool)
                with np.errstate(invalid="ignore"):
                    over = ~(p[:, ~half].sum(axis=1, dtype=np.float32) <= bound)
                    over |= ~(p[:, half].sum(axis=1, dtype=np.float32) <= bound)
                moved = np.isin(group, np.unique(group[over]))
                if moved.any():
                    m_new = np.where(moved, np.maximum(m, m_cand), m).astype(np.float32)
                    with np.errstate(invalid="ignore"):
                        alpha = np.where(m_new == m, np.float32(1.0),
                                         np.exp2((m - m_new).astype(np.float32))).astype(np.float32)
                    l = (l * alpha).astype(np.float32)
                    acc *= alpha[:, None].astype(np.float64)
                    m = m_new
                    p = exps(st, m)
            else:
                upd = m_cand > (m + thr)
                m_new = np.where(upd, m_cand, m)
                with np.errstate(invalid="ignore"):
                    alpha = np.where(upd, np.exp2((m - m_new).astype(np.float32)), np.float32(1.0)).astype(np.float32)
                l = (l * alpha).astype(np.float32)
                acc *= alpha[:, None].astype(np.float64)
                m = m_new
                p = exps(st, m)
            l = (l + p.sum(axis=1, dtype=np.float32)).astype(np.float32)
            pr = round_e5m2(p) if round_p else p
            acc += pr.astype(np.float64) @ vf[i, lo:hi]
        out[i] = (acc * (1.0 / l.astype(np.float64))[:, None]).astype(np.float32)
        with np.errstate(divide="ignore"):
            lse[i] = ((m + np.log2(l)) * np.float32(LN2)).astype(np.float32)
    out = out.reshape(*lead, sq, vf.shape[-1])
    lse = lse.reshape(*lead, sq)
    return round_to(out, out_dtype), lse


def _causal_mask(sq: int, sk: int) -> np.ndarray:
    # True where the key is masked: triu(ones(sq, sk), diagonal=1), as in
    # evaluate_attention.py:137-140.
    return np.triu(np.ones((sq, sk), dtype=bool), k=1)


def attention_ref(q, k, v, causal: bool, sm_scale: float, out_dtype: str | None = None,
                  compute_dtype=np.float32):
    """fp32 softmax(sm_scale * q k^T [+ causal mask]) v and the natural-log LSE.

    q: [..., Sq, D], k, v: [..., Sk, D] (any leading batch/head dims), holding
    the exact values of the fp16/bf16 inputs as float32.  Returns
    (out, lse): out [..., Sq, D] rounded to `out_dtype` (float32 values),
    lse [..., Sq] float32.  Heads are processed one at a time, so memory stays
    O(Sq * Sk) per head.
    """
    q = np.asarray(q, dtype=np.float32)
    k = np.asarray(k, dtype=np.float32)
    v = np.asarray(v, dtype=np.float32)
    if q.ndim < 2 or k.shape[:-2] != q.shape[:-2] or v.shape[:-1] != k.shape[:-1]:
        raise ValueError("q, k, v must share leading dims; k and v must share Sk")
    if q.shape[-1] != k.shape[-1]:
        raise ValueError("q and k must share the head dim")
    lead = q.shape[:-2]
    sq, d = q.shape[-2:]
    sk = k.shape[-2]
    dv = v.shape[-1]
    qf = q.reshape(-1, sq, d)
    kf = k.reshape(-1, sk, d)
    vf = v.reshape(-1, sk, dv)
    out = np.empty((qf.shape[0], sq, dv), dtype=np.float32)
    lse = np.empty((qf.shape[0], sq), dtype=np.float32)
    mask = _causal_mask(sq, sk) if causal else None
    ct = compute_dtype
    for i in range(qf.shape[0]):
        scores = (qf[i].astype(ct) @ kf[i].astype(ct).T) * ct(sm_scale)
        if mask is not None:
            scores = np.where(mask, ct(-np.inf), scores)
        row_max = scores.max(axis=-1, keepdims=True)
        # Rows with no visible key (only possible when Sq > Sk is not the
        # case for top-left causal) would give -inf max; keep them finite.
        safe_max = np.where(np.isfinite(row_max), row_max, ct(0))
        e = np.exp(scores - safe_max)
        denom = e.sum(axis=-1, keepdims=True)
        probs = e / denom
        out[i] = (probs @ vf[i].astype(ct)).astype(np.float32)
        lse[i] = (np.log(denom[..., 0]) + safe_max[..., 0]).astype(np.float32)
    out = out.reshape(*lead, sq, dv)
    lse = lse.reshape(*lead, sq)
    return round_to(out, out_dtype), lse


def attention_bruteforce(q, k, v, causal: bool, sm_scale: float):
    """Row-by-row float64 restatement with explicit loops (tiny inputs only).

    For each query row i: logits s_j = sm_scale * sum_d q[i,d] k[j,d] over the
    visible keys j (j <= i when causal), m = max_j s_j,
    lse = m + log(sum_j exp(s_j - m)), out[i, :] = sum_j exp(s_j - lse) v[j, :].
    q, k, v: [Sq, D], [Sk, D], [Sk, Dv].  Returns float64 (out, lse).
    """
    q = np.asarray(q, dtype=np.float64)
    k = np.asarray(k, dtype=np.float64)
    v = np.asarray(v, dtype=np.float64)
    sq, d = q.shape
    sk = k.shape[0]
    out = np.zeros((sq, v.shape[1]), dtype=np.float64)
    lse = np.zeros(sq, dtype=np.float64)
    for i in range(sq):
        last = min(i, sk - 1) if causal else sk - 1
        logits = []
        for j in range(last + 1):
            acc = 0.0
            for t in range(d):
                acc += q[i, t] * k[j, t]
            logits.append(sm_scale * acc)
        m = max(logits)
        total = 0.0
        for s in logits:
            total += math.exp(s - m)
        lse[i] = m + math.log(total)
        for j, s in enumerate(logits):
            w = math.exp(s - lse[i])
            for t in range(v.shape[1]):
                out[i, t] += w * v[j, t]
    return out, lse


def attention_partial(q, k, v, causal: bool, sm_scale: float, lo: int, hi: int):
    """Attention over keys [lo, hi) only: (O_part float32, LSE_part float32).

    Same shapes and causal convention as attention_ref (key j visible to query
    i iff j <= i); O_part is normalised by the range's own row sum; rows that
    see no key of the range get O_part = 0 and LSE_part = -inf.
    """
    q = np.asarray(q, dtype=np.float32)
    k = np.asarray(k, dtype=np.float32)
    v = np.asarray(v, dtype=np.float32)
    sq, sk = q.shape[-2], k.shape[-2]
    lead = q.shape[:-2]
    qf = q.reshape(-1, sq, q.shape[-1])
    kf = k.reshape(-1, sk, k.shape[-1])
    vf = v.reshape(-1, sk, v.shape[-1])
    out = np.zeros((qf.shape[0], sq, vf.shape[-1]), dtype=np.float32)
    lse = np.full((qf.shape[0], sq), -np.inf, dtype=np.float32)
    keys = np.arange(lo, min(hi, sk))
    if keys.size == 0:
        return out.reshape(*lead, sq, -1), lse.reshape(*lead, sq)
    visible = np.ones((sq, keys.size), dtype=bool)
    if causal:
        visible = keys[None, :] <= np.arange(sq)[:, None]
    for i in range(qf.shape[0]):
        scores = (qf[i] @ kf[i][keys].T) * np.float32(sm_scale)
        scores = np.where(visible, scores, np.float32(-np.inf))
        row_max = scores.max(axis=-1, keepdims=True)
        seen = np.isfinite(row_max[..., 0])
        safe_max = np.where(np.isfinite(row_max), row_max, np.float32(0))
        e = np.exp(scores - safe_max)
        denom = e.sum(axis=-1, keepdims=True)
        o = (e / np.where(denom > 0, denom, 1)) @ vf[i][keys]
        out[i] = np.where(seen[:, None], o, 0).astype(np.float32)
        lse[i] = np.where(seen, np.log(np.where(denom[..., 0] > 0, denom[..., 0], 1)) + safe_max[..., 0],
                          -np.inf).astype(np.float32)
    return out.reshape(*lead, sq, -1), lse.reshape(*lead, sq)


def merge_partials(parts):
    """Exact LSE-weighted merge of [(O_s, LSE_s), ...] -> (O, LSE), float32.

    m = max_s LSE_s;  w_s = exp(LSE_s - m) (0 where LSE_s = -inf);
    LSE = m + log(sum_s w_s);  O = sum_s w_s O_s / sum_s w_s.
    """
    lses = np.stack([np.asarray(l, dtype=np.float64) for _, l in parts])
    outs = np.stack([np.asarray(o, dtype=np.float64) for o, _ in parts])
    m = lses.max(axis=0)
    safe_m = np.where(np.isfinite(m), m, 0.0)
    w = np.where(np.isfinite(lses), np.exp(lses - safe_m), 0.0)
    wsum = w.sum(axis=0)
    o = (w[..., None] * outs).sum(axis=0) / np.where(wsum > 0, wsum, 1.0)[..., None]
    lse = np.where(wsum > 0, safe_m + np.log(np.where(wsum > 0, wsum, 1.0)), -np.inf)
    return o.astype(np.float32), lse.astype(np.float32)


def attention_flops(b: int, h: int, sq: int, sk: int, d: int, causal: bool) -> float:
    """Algorithmic FLOPs of one forward: 4*B*H*Sq*Sk*D, halved when causal."""
    f = 4.0 * b * h * sq * sk * d
    return f / 2.0 if causal else f
