"""Numerical model of the e4m3-MFMA history kernels (CPU, numpy).

TEST INFRASTRUCTURE ONLY (see ``oracle/__init__.py``).  Parity of the HIP
path is judged against the float64 attention of ``oracle.pcp_oracle``
(reference.py:16-32 restated).  This module answers a different question:
what a kernel that rounds Q and the probabilities P to e4m3 *should* output,
bit for bit up to fp32 accumulation order, so that a test can tell the
method's own rounding error (inherent to e4m3 operands, larger when few keys
carry the softmax) from a kernel bug.  It follows the kernels' arithmetic:

* Q rows quantised to e4m3 per row: ``e4m3(q * (448 / amax))`` in fp32, the
  score factor ``amax / 448 * softmax_scale * k_scale * log2(e)`` (fp32);
* raw scores ``sum_d q8_d k8_d`` of the e4m3 codes (the MFMA's products are
  exact), rounded to fp32;
* the walk over the block table in entry order (rank-major), a page's valid
  prefix in 64-key tiles, entries with no valid token or an out-of-range
  page skipped;
* the online softmax of each kernel:

  - ``overlap`` (e4m3 MFMAs at head_dim 256): per row and tile, reference
    ``m = max(m, tile_max * c - 2.5)`` from a floor of -1e30; probabilities
    ``2^(s c - m + 6)`` rounded to e4m3, either as the code
    ``round(8 x + 56)`` of the linear-mantissa exp2 (``exp2="fast"``) or as
    ``e4m3(2^x)`` (``"exact"``);
  - ``tile`` (e4m3 MFMAs at head_dim 64/128): per row, the reference starts
    at -inf and moves to ``tile_max * c`` when that exceeds it by more than
    2.5; probabilities ``e4m3(2^(s c - m + 6))``;

  with the row sum ``l`` taken over the rounded probabilities and both ``l``
  and ``O`` rescaled by ``2^(m_old - m_new)``;
* ``O * v_scale / l`` (the kernel rounds it to bf16; the model returns
  float64), and the log-sum-exp ``ln l + (m - 6) ln 2`` less 0.03987 for the
  fast exp2;
* split launches: each range of table entries ``[E s / S, E (s + 1) / S)``
  normalised on its own and merged by log-sum-exp.

Pinned in tests/test_e4m3_model.py: with both roundings switched off it is
float64 attention (``oracle.pcp_oracle``) to 1e-12; a scalar per-row loop
written independently gives identical numbers; identical keys give the mean
of V exactly and a dominant key its V; the fast code decodes to the
linear interpolation of 2^x between powers of two.
"""

from __future__ import annotations

import numpy as np

from .pcp_oracle import E4M3FN_DECODE, decode_bfloat16

KEY_TILE = 64
P_BIAS_LOG2 = 6.0
MAX_FLOOR = np.float32(-1.0e30)
FAST_LSE_BIAS = 0.03987
LOG2E = np.float32(1.4426950408889634)
FP8_MAX = np.float32(448.0)


def round_e4m3(x: np.ndarray) -> np.ndarray:
    """Round to the nearest e4m3fn value (ties to even), as float64.

    Magnitudes up to 464 round to 448 (an fp32 product meant to be 448 can
    come out an ulp above it); beyond that e4m3fn has no value, and the
    kernels never go there.
    """
    x = np.asarray(x, dtype=np.float64)
    a = np.abs(x)
    if np.any(a[np.isfinite(a)] >= 464.0):
        raise ValueError("value at or beyond 464, which e4m3fn cannot hold")
    with np.errstate(divide="ignore"):
        e = np.floor(np.log2(np.where(a > 0, a, 1.0)))
    e = np.maximum(e, -6.0)  # subnormals share the 2^-9 step of the smallest binade
    step = np.exp2(e - 3.0)
    r = np.minimum(np.rint(a / step) * step, 448.0)
    return np.copysign(r, x)


def fast_exp2_code(x: np.ndarray) -> np.ndarray:
    """e4m3 code ``clamp(round_even(8 x + 56), 0, 255)`` of 2^x's linear-mantissa form (float64 x)."""
    y = np.asarray(x, dtype=np.float64) * 8.0 + 56.0
    return np.clip(np.rint(y), 0, 255).astype(np.uint8)


def _f32(x):
    return np.asarray(x, dtype=np.float64).astype(np.float32)


def quantise_q_rows(q_bits: np.ndarray) -> tuple[np.ndarray, np.ndarray]:
    """Rows of bf16 bits ``[R, D]`` -> (e4m3 values float64 ``[R, D]``, sigma fp32 ``[R]``)."""
    q = decode_bfloat16(q_bits).astype(np.float32)
    amax = np.abs(q).max(axis=1)
    pos = amax > 0
    inv = np.where(pos, FP8_MAX / np.where(pos, amax, 1), np.float32(1)).astype(np.float32)
    sigma = np.where(pos, amax / FP8_MAX, np.float32(1)).astype(np.float32)
    q8 = round_e4m3((q * inv[:, None]).astype(np.float32))
    return q8, sigma


def walk_pages(block_table: np.ndarray, page_valid_len: np.ndarray, num_pages: int, block_size: int,
               entries: tuple[int, int] | None = None) -> list[tuple[int, int]]:
    """(page, valid length) of the entries the kernels visit, in walk order."""
    table = np.asarray(block_table).reshape(-1)
    lens = np.asarray(page_valid_len).reshape(-1)
    lo, hi = entries if entries is not None else (0, table.size)
    out = []
    for e in range(lo, hi):
        n = min(int(lens[e]), block_size)
        page = int(table[e])
        if n > 0 and 0 <= page < num_pages:
            out.append((page, n))
    return out


def _tiles(walk: list[tuple[int, int]]) -> list[tuple[int, int, int]]:
    """(page, first key, keys) of every 64-key tile of the walk."""
    return [(page, base, min(KEY_TILE, n - base)) for page, n in walk for base in range(0, n, KEY_TILE)]


def _softmax_walk(scores, v_tiles, tiles, cscale, kernel, exp2, q_round=True, p_round=True):
    """Online softmax over the tiles for rows sharing one KV head.

    scores: fp32 raw scores ``[R, keys]`` in walk order; v_tiles: float64
    V rows ``[keys, D]`` in the same order; cscale: fp32 ``[R]``.  Returns
    (O float64 [R, D] un-normalised, l float64 [R], m fp32 [R]).
    """
    rows = scores.shape[0]
    d = v_tiles.shape[1]
    o = np.zeros((rows, d))
    l = np.zeros(rows)
    m = np.full(rows, MAX_FLOOR if kernel == "overlap" else -np.inf, dtype=np.float32)
    cscale = cscale.astype(np.float32)
    key = 0
    for _, _, n in tiles:
        s = scores[:, key:key + n]
        vt = v_tiles[key:key + n]
        key += n
        mxs = (s.max(axis=1).astype(np.float32) * cscale).astype(np.float32)
        if kernel == "overlap":
            m_new = np.maximum(m, (mxs - np.float32(2.5)).astype(np.float32))
        else:
            m_new = np.where(mxs > (m + np.float32(2.5)), mxs, m).astype(np.float32)
        with np.errstate(invalid="ignore"):
            alpha = np.exp2((m - m_new).astype(np.float32).astype(np.float64))
        alpha = np.where(np.isnan(alpha), 0.0, alpha)
        m = m_new
        if kernel == "overlap" and exp2 == "fast" and p_round:
            cscale8 = (np.float32(8) * cscale).astype(np.float32)
            shift = _f32(-8.0 * m.astype(np.float64) + (8.0 * P_BIAS_LOG2 + 56.0))
            # fma(s, 8 c, 8 (6 - m) + 56) = 8 x + 56, rounded to an integer code
            arg = _f32(s.astype(np.float64) * cscale8[:, None] + shift[:, None])
            p = E4M3FN_DECODE[np.clip(np.rint(arg.astype(np.float64)), 0, 255).astype(np.uint8)]
        else:
            shift = _f32(P_BIAS_LOG2 - m.astype(np.float64))
            arg = _f32(s.astype(np.float64) * cscale[:, None] + shift[:, None])
            p = np.exp2(arg.astype(np.float64))
            if p_round:
                p = round_e4m3(_f32(p))
        p = np.where(np.isfinite(s), p, 0.0)
        o = o * alpha[:, None] + p @ vt
        l = l * alpha + p.sum(axis=1)
    return o, l, m


GUARD_MIN_MASS = 384.0
VSTATS_KEYS = 2048


def guard_thresholds(pool_codes, block_table, page_valid_len, *, num_kv_heads, block_size, head_dim, v_scale=1.0):
    """The precision guard's probability-mass threshold per KV head.

    ``GUARD_MIN_MASS * v_scale^2 * max_d Var(V[h, :, d])``: the population
    variance per channel of the e4m3 V codes of head h over the keys the
    walk visits, sampled as the kernels' statistics do (every s-th key of
    each page's valid prefix, s the smallest power of two with valid keys /
    s <= VSTATS_KEYS).  A row whose mass ``sum_k 2^(x_k - m)`` is below it is
    recomputed with BF16 MFMAs.  The rounding error of e4m3 Q and P in a row
    grows as the spread of the V values it averages over sqrt(mass), so the
    threshold grows with the variance; 384 is where unit-variance V keeps
    the e4m3 rows within about half the 2e-2 bar.
    """
    pool = E4M3FN_DECODE[np.asarray(pool_codes, dtype=np.uint8)].reshape(-1, 2, num_kv_heads, block_size, head_dim)
    walk = walk_pages(block_table, page_valid_len, pool.shape[0], block_size)
    total = sum(n for _, n in walk)
    stride = 1
    while total // stride > VSTATS_KEYS:
        stride *= 2
    thr = np.zeros(num_kv_heads)
    for h in range(num_kv_heads):
        if not walk:
            continue
        vals = np.concatenate([pool[page, 1, h, 0:n:stride] for page, n in walk])
        thr[h] = GUARD_MIN_MASS * v_scale ** 2 * vals.var(axis=0).max()
    return thr


def emulate_rows(q_bits, pool_codes, block_table, page_valid_len, *, num_kv_heads, block_size, softmax_scale,
                 k_scale=1.0, v_scale=1.0, kernel="overlap", exp2="fast", splits=1, rows=None, q_round=True,
                 p_round=True, chunk_rows=256, return_mass=False):
    """Model outputs and log-sum-exps of query rows.

    ``q_bits``: uint16 bf16 bits ``[pcp, Hq, local_q, D]`` (the stacked Q);
    ``pool_codes``: uint8 e4m3 codes ``[num_pages, 2 * Hkv * block * D]``;
    ``block_table``/``page_valid_len``: int ``[pcp, max_local_blocks]``.
    ``rows``: ``None`` for every row (returns out float64 ``[pcp, Hq,
    local_q, D]`` and lse ``[pcp, Hq, local_q]``), or an int array of
    ``(rank, q_head, token)`` triples (returns ``[n, D]`` and ``[n]``).  ``q_round``/``p_round`` switch the two roundings
    off (the model is then plain float64 attention up to fp32 factors).

    ``return_mass``: also return each row's probability mass ``l / 2^6``, the
    sum of ``2^(score - m)`` over its keys against the kernel's final
    reference max ``m`` (which trails the true maximum by at most 2.5); split
    launches sum every range's mass against the largest range reference.
    This is the quantity the kernels' precision guard tests.
    """
    if kernel not in ("overlap", "tile") or exp2 not in ("fast", "exact"):
        raise ValueError("kernel must be 'overlap' or 'tile', exp2 'fast' or 'exact'")
    q_bits = np.asarray(q_bits, dtype=np.uint16)
    pcp, hq, lq, d = q_bits.shape
    group = hq // num_kv_heads
    pool = E4M3FN_DECODE[np.asarray(pool_codes, dtype=np.uint8)].reshape(-1, 2, num_kv_heads, block_size, d)
    num_pages = pool.shape[0]
    entries = np.asarray(block_table).size
    score_scale = np.float32(np.float32(np.float32(softmax_scale) * np.float32(k_scale)) * LOG2E)
    fast = kernel == "overlap" and exp2 == "fast" and p_round
    bias = FAST_LSE_BIAS if fast else 0.0
    ranges = [(entries * s_idx // splits, entries * (s_idx + 1) // splits) for s_idx in range(splits)]
    walks = [_tiles(walk_pages(block_table, page_valid_len, num_pages, block_size, r)) for r in ranges]

    # row index within KV head g (the kernels' order): rank, head in group, token
    def head_row(rank, qh, tok):
        return (rank * group + qh % group) * lq + tok

    if rows is None:
        wanted = [(g, np.arange(pcp * group * lq)) for g in range(num_kv_heads)]
    else:
        rows = np.asarray(rows, dtype=np.int64).reshape(-1, 3)
        wanted = []
        for g in range(num_kv_heads):
            sel = rows[:, 1] // group == g
            if sel.any():
                wanted.append((g, np.unique(head_row(rows[sel, 0], rows[sel, 1], rows[sel, 2]))))
    results = {}
    for g, head_rows in wanted:
        allbits = q_bits[:, g * group:(g + 1) * group].reshape(-1, d)
        for c0 in range(0, head_rows.size, chunk_rows):
            idx = head_rows[c0:c0 + chunk_rows]
            rbits = allbits[idx]
            if q_round:
                q8, sigma = quantise_q_rows(rbits)
            else:
                q8, sigma = decode_bfloat16(rbits), np.ones(rbits.shape[0], dtype=np.float32)
            cscale = (sigma * score_scale).astype(np.float32)
            parts = []
            for tiles in walks:
                if not tiles:
                    parts.append((np.zeros((idx.size, d)), np.full(idx.size, -np.inf), np.zeros(idx.size),
                                  np.full(idx.size, -np.inf)))
                    continue
                keys = np.concatenate([pool[p, 0, g, b:b + n] for p, b, n in tiles])
                vals = np.concatenate([pool[p, 1, g, b:b + n] for p, b, n in tiles])
                scores = _f32(q8 @ keys.T)
                o, l, m = _softmax_walk(scores, vals, tiles, cscale, kernel, exp2, q_round, p_round)
                with np.errstate(divide="ignore", invalid="ignore"):
                    part_out = np.where(l[:, None] > 0, o * (v_scale / l)[:, None], 0.0)
                    part_lse = np.where(l > 0, np.log(l) + (m.astype(np.float64) - P_BIAS_LOG2) * np.log(2.0) - bias,
                                        -np.inf)
                parts.append((part_out, part_lse, l, m.astype(np.float64)))
            if splits == 1:
                res, res_lse = parts[0][:2]
                res_mass = parts[0][2] / 2.0 ** P_BIAS_LOG2
            else:
                lses = np.stack([p[1] for p in parts])
                mx = lses.max(axis=0)
                with np.errstate(invalid="ignore"):
                    w = np.where(np.isfinite(lses), np.exp(lses - np.where(np.isfinite(mx), mx, 0.0)), 0.0)
                wsum = w.sum(axis=0)
                safe = np.where(wsum > 0, wsum, 1.0)
                res = np.where(wsum[:, None] > 0,
                               np.einsum("sr,srd->rd", w, np.stack([p[0] for p in parts])) / safe[:, None], 0.0)
                res_lse = np.where(wsum > 0, mx + np.log(safe), -np.inf)
                m_ref = np.stack([p[3] for p in parts]).max(axis=0)
                res_mass = sum(np.where(p[2] > 0, p[2] * np.exp2(p[3] - m_ref), 0.0) for p in parts) / 2.0 ** P_BIAS_LOG2
            for i, r in enumerate(idx.tolist()):
                results[(g, r)] = (res[i], res_lse[i], res_mass[i])
    if rows is None:
        out = np.zeros((pcp, hq, lq, d))
        lse = np.full((pcp, hq, lq), -np.inf)
        mass = np.zeros((pcp, hq, lq))
        for (g, r), (o_row, l_row, w_row) in results.items():
            rank, rem = divmod(r, group * lq)
            hig, tok = divmod(rem, lq)
            out[rank, g * group + hig, tok] = o_row
            lse[rank, g * group + hig, tok] = l_row
            mass[rank, g * group + hig, tok] = w_row
    else:
        keys = [(int(qh) // group, int(head_row(rank, qh, tok))) for rank, qh, tok in rows]
        out = np.stack([results[k][0] for k in keys])
        lse = np.array([results[k][1] for k in keys])
        mass = np.array([results[k][2] for k in keys])
    return (out, lse, mass) if return_mass else (out, lse)
