"""numpy float64 restatement of the reference's causal attention math -- TEST INFRASTRUCTURE ONLY.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg use this
module, and only as the checker.  Every function cites the reference lines it
follows; tests/test_oracle.py pins each one independently (see oracle/__init__.py).

Shapes: q [B, H, N, D]; k, v [B, H_kv, N, D] with H_kv dividing H.
"""

import math

import numpy as np

LOG2E = 1.4426950408889634  # attention/fused/fused.py:9


def _f64(x):
    return np.asarray(x, dtype=np.float64)


def expand_kv(k, v, num_q_heads):
    """Repeat each K/V head so query head h uses K/V head h // (H // H_kv).

    attention/gqa/reference_gqa.py:15-26 (repeat_interleave along the head axis)."""
    H_kv = k.shape[1]
    if v.shape[1] != H_kv:
        raise ValueError(f"K/V head count mismatch: K={H_kv}, V={v.shape[1]}")
    if H_kv < 1 or num_q_heads % H_kv != 0:
        raise ValueError(f"H={num_q_heads} not divisible by H_kv={H_kv}")
    group = num_q_heads // H_kv
    return np.repeat(k, group, axis=1), np.repeat(v, group, axis=1)


def masked_scores(q, k, rows=None):
    """S = Q K^T / sqrt(D) with -inf where key > query (attention/fused/reference.py:19-21).

    rows: optional 1-D array of query rows to evaluate (rows are independent)."""
    q, k = _f64(q), _f64(k)
    k, _ = expand_kv(k, k, q.shape[1])
    N, D = k.shape[2], q.shape[3]
    if rows is None:
        rows = np.arange(q.shape[2])
    rows = np.asarray(rows)
    s = (q[:, :, rows, :] @ np.swapaxes(k, -1, -2)) / math.sqrt(D)
    future = np.arange(N)[None, :] > rows[:, None]
    s[..., future] = -np.inf
    return s


def probs(q, k, rows=None):
    """P = softmax(S) over keys (attention/fused/reference.py:22), max-subtracted."""
    s = masked_scores(q, k, rows)
    m = s.max(axis=-1, keepdims=True)
    e = np.exp(s - m)
    return e / e.sum(axis=-1, keepdims=True)


def forward(q, k, v, rows=None):
    """O = softmax(Q K^T / sqrt(D) + causal) V.

    attention/fused/reference.py:16-23; GQA via attention/gqa/reference_gqa.py:35-43."""
    v = _f64(v)
    _, v = expand_kv(v, v, q.shape[1])
    return probs(q, k, rows) @ v


def lse_log2(q, k, rows=None):
    """Per-row LSE in the reference's units: m + log2(l) for scores scaled by log2(e)/sqrt(D).

    attention/backward/fused_backward.py:61-62 (m, l) and :169 (lse = m + log2(l)).
    Equals the natural-log logsumexp of S/sqrt(D) times log2(e)."""
    s = masked_scores(q, k, rows) * LOG2E
    m = s.max(axis=-1, keepdims=True)
    return (m + np.log2(np.exp2(s - m).sum(axis=-1, keepdims=True)))[..., 0]


def delta(do, o):
    """Delta = rowsum(dO * O) in float64 (attention/backward/fused_backward.py:175)."""
    return (_f64(do) * _f64(o)).sum(axis=-1)


def backward(q, k, v, do):
    """Closed-form gradients of O = softmax(QK^T/sqrt(D) + causal) V (report p.10 eq. 5).

    dV = P^T dO, dP = dO V^T, dS = P * (dP - Delta), dQ = dS K / sqrt(D), dK = dS^T Q / sqrt(D)
    (the quantities of attention/backward/fused_backward.py:92-107, 135-147).
    For GQA the K/V gradients of a group's query heads are summed onto their K/V head."""
    q, k, v, do = _f64(q), _f64(k), _f64(v), _f64(do)
    B, H, N, D = q.shape
    H_kv = k.shape[1]
    ke, ve = expand_kv(k, v, H)
    p = probs(q, k)
    o = p @ ve
    dv = np.swapaxes(p, -1, -2) @ do
    dp = do @ np.swapaxes(ve, -1, -2)
    ds = p * (dp - delta(do, o)[..., None])
    dq = ds @ ke / math.sqrt(D)
    dk = np.swapaxes(ds, -1, -2) @ q / math.sqrt(D)
    g = H // H_kv
    dk = dk.reshape(B, H_kv, g, N, D).sum(axis=2)
    dv = dv.reshape(B, H_kv, g, N, D).sum(axis=2)
    return o, dq, dk, dv


def dq_rows(q, k, v, do, rows):
    """dQ for a subset of query rows (rows are independent): dQ_r = sum_j dS_rj K_j / sqrt(D)."""
    q, k, v, do = _f64(q), _f64(k), _f64(v), _f64(do)
    D = q.shape[3]
    ke, ve = expand_kv(k, v, q.shape[1])
    p = probs(q, k, rows)
    o = p @ ve
    dor = do[:, :, rows, :]
    dp = dor @ np.swapaxes(ve, -1, -2)
    ds = p * (dp - delta(dor, o)[..., None])
    return ds @ ke / math.sqrt(D)


def online_softmax_forward(q, k, v, tile_m, tile_n):
    """Tile-by-tile online softmax exactly as the fused kernel's loop, in float64.

    attention/fused/fused.py:11-65: heavy-first query tiles, causal tile bounds
    (:30,32), mask on straddling tiles (:45-47), running max in scaled log2 units
    (:50), alpha = exp2(m - m_new) (:53), p = exp2(s*c - m_new) (:56),
    l = l*alpha + rowsum(p) (:59), acc = acc*alpha + p.v (:60), O = acc / l (:64).
    Returns (O, lse) with lse = m + log2(l) (attention/backward/fused_backward.py:169)."""
    q, k, v = _f64(q), _f64(k), _f64(v)
    B, H, N, D = q.shape
    k, v = expand_kv(k, v, H)
    c = LOG2E / math.sqrt(D)
    out = np.empty_like(q)
    lse = np.empty((B, H, N))
    n_q = N // tile_m
    for i in reversed(range(n_q)):  # heaviest (last) query tile first
        rows = i * tile_m + np.arange(tile_m)
        qi = q[:, :, rows, :]
        m = np.full((B, H, tile_m, 1), -np.inf)
        l = np.zeros((B, H, tile_m, 1))
        acc = np.zeros((B, H, tile_m, D))
        num_kv = ((i + 1) * tile_m + tile_n - 1) // tile_n
        mask_start = (i * tile_m) // tile_n
        for j in range(num_kv):
            cols = j * tile_n + np.arange(tile_n)
            s = qi @ np.swapaxes(k[:, :, cols, :], -1, -2)
            if j >= mask_start:
                s = np.where(cols[None, :] > rows[:, None], -np.inf, s)
            m_new = np.maximum(m, s.max(axis=-1, keepdims=True) * c)
            alpha = np.exp2(m - m_new)
            p = np.exp2(s * c - m_new)
            l = l * alpha + p.sum(axis=-1, keepdims=True)
            acc = acc * alpha + p @ v[:, :, cols, :]
            m = m_new
        out[:, :, rows, :] = acc / l
        lse[:, :, rows] = (m + np.log2(l))[..., 0]
    return out, lse


def naive_loops(q, k, v):
    """Pure-Python per-element causal attention for tiny inputs (independent of numpy's
    vectorised paths): for each row r, weights exp(s_rj - max) over j <= r."""
    q, k, v = _f64(q), _f64(k), _f64(v)
    B, H, N, D = q.shape
    group = H // k.shape[1]
    out = np.zeros((B, H, N, D))
    inv = 1.0 / math.sqrt(D)
    for b in range(B):
        for h in range(H):
            hk = h // group
            for r in range(N):
                sc = []
                for j in range(r + 1):
                    acc = 0.0
                    for d in range(D):
                        acc += q[b, h, r, d] * k[b, hk, j, d]
                    sc.append(acc * inv)
                mx = max(sc)
                w = [math.exp(x - mx) for x in sc]
                tot = sum(w)
                for d in range(D):
                    out[b, h, r, d] = sum(w[j] * v[b, hk, j, d] for j in range(r + 1)) / tot
    return out


def sample_rows(N, tile=64, count=48, seed=0):
    """Deterministic query rows covering the edges that matter: the first rows (few keys),
    tile boundaries, the last row, and random interior rows."""
    rng = np.random.default_rng(seed)
    fixed = {0, 1, 2, 31, 32, 33, 63, N - 1, N - 2, N // 2}
    for t in (64, 128):
        for base in (t, 2 * t, N - t):
            fixed.update({base - 1, base})
    fixed = {r for r in fixed if 0 <= r < N}
    extra = rng.choice(N, size=min(N, max(0, count - len(fixed))), replace=False)
    return np.array(sorted(fixed.union(int(x) for x in extra)))
