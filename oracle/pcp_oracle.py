"""CPU restatement of the reference's PCP attention specification.

TEST INFRASTRUCTURE ONLY (see ``oracle/__init__.py``): imported by tests,
``__graft_entry__.smoke()`` and ``bench.py``'s CPU baseline, never by the
product.

Each function cites the reference file:line it restates.  How each one is
pinned (tests/test_oracle.py):

* e4m3 decode table - built from the OCP e4m3fn bit definition, checked on
  all 256 codes against torch's float8_e4m3fn and against hand-known values.
* index maps (owner/local position, positions per rank, shard/gather, pack,
  block mask) - the reference tests' known answers (tests/test_layout.py,
  test_kernel_pack.py, test_runner.py), the README closed form checked by
  brute-force enumeration, and the hand-worked table in
  tests/golden/owner_pcp3_il2.json.
* dense attention - float64; checked against a per-row brute-force loop, a
  closed form (identical keys give the mean of V) and one-hot limits.
* ring model - equals dense attention (tests/test_reference.py:8-56 in the
  reference) and its loop order is checked on a tiny case by recording the
  visited (rank, block, source rank) sequence.
* per-rank valid length for unaligned histories - brute force over global
  positions with owner_and_local_position.
* attention with log-sum-exp and per-row key limits (current-token causal
  attention, merged with the history) - the lse against a per-row
  ``math.fsum`` loop and the closed form ``c + ln n`` of n identical scores;
  the causal and history-plus-current outputs against torch's
  ``scaled_dot_product_attention`` (float64, is_causal / an explicit boolean
  mask over the concatenated keys) on global-order queries, which also pins
  the inverse of the striping.  The reference has no current-token
  attention (README.md:17-18): these follow the standard causal definition.
"""

from __future__ import annotations

from dataclasses import dataclass
from math import ceil, sqrt

import numpy as np

# ---------------------------------------------------------------------------
# FP8 e4m3fn decode (OCP "fn" variant: bias 7, no infinities, S.1111.111 NaN).
# ---------------------------------------------------------------------------


def _build_e4m3fn_table() -> np.ndarray:
    table = np.empty(256, dtype=np.float64)
    for code in range(256):
        sign = -1.0 if code & 0x80 else 1.0
        exponent = (code >> 3) & 0xF
        mantissa = code & 0x7
        if exponent == 0xF and mantissa == 0x7:
            table[code] = np.nan
        elif exponent == 0:
            table[code] = sign * mantissa * 2.0 ** -9
        else:
            table[code] = sign * (1.0 + mantissa / 8.0) * 2.0 ** (exponent - 7)
    return table


E4M3FN_DECODE = _build_e4m3fn_table()


def decode_e4m3fn(codes: np.ndarray) -> np.ndarray:
    """float64 values of uint8 e4m3fn codes."""
    return E4M3FN_DECODE[np.asarray(codes, dtype=np.uint8)]


def decode_bfloat16(bits: np.ndarray) -> np.ndarray:
    """float64 values of uint16 bfloat16 bit patterns."""
    wide = np.asarray(bits, dtype=np.uint16).astype(np.uint32) << 16
    return wide.view(np.float32).astype(np.float64)


# ---------------------------------------------------------------------------
# Shape maths (config.py:29-59).
# ---------------------------------------------------------------------------


@dataclass(frozen=True)
class OracleShape:
    pcp_size: int
    current_len: int
    max_history_len: int
    actual_history_len: int
    block_size: int
    interleave_size: int
    num_q_heads: int
    num_kv_heads: int
    head_dim: int

    @classmethod
    def from_config(cls, config) -> "OracleShape":
        return cls(*(int(getattr(config, f)) for f in cls.__dataclass_fields__))

    @property
    def softmax_scale(self) -> float:  # config.py:30-31
        return 1.0 / sqrt(self.head_dim)

    @property
    def group(self) -> int:  # config.py:34-35
        return self.num_q_heads // self.num_kv_heads

    @property
    def local_q_len(self) -> int:  # config.py:38-39
        return self.current_len // self.pcp_size

    @property
    def max_local_history_len(self) -> int:  # config.py:42-43
        return self.max_history_len // self.pcp_size

    @property
    def max_local_blocks(self) -> int:  # config.py:50-51
        return ceil(self.max_local_history_len / self.block_size)

    def rank_history_len(self, rank: int) -> int:
        """Tokens ``p < actual_history_len`` owned by ``rank`` (brute-force pinned)."""
        stride = self.pcp_size * self.interleave_size
        full, tail = divmod(self.actual_history_len, stride)
        extra = tail - rank * self.interleave_size
        return full * self.interleave_size + max(0, min(self.interleave_size, extra))

    @property
    def actual_local_history_len(self) -> int:  # config.py:46-47 for aligned lengths
        return self.rank_history_len(0)

    @property
    def actual_local_blocks(self) -> int:  # config.py:54-55
        return ceil(self.actual_local_history_len / self.block_size)


# ---------------------------------------------------------------------------
# Striped layout (layout.py:10-132, README.md:22-29).
# ---------------------------------------------------------------------------


def owner_and_local_position(p: int, pcp_size: int, interleave_size: int) -> tuple[int, int]:
    """layout.py:10-16: chunk = p // il; owner = chunk % pcp; local = (chunk // pcp) * il + p % il."""
    chunk, within = divmod(p, interleave_size)
    return chunk % pcp_size, (chunk // pcp_size) * interleave_size + within


def global_positions(total_len: int, rank: int, pcp_size: int, interleave_size: int) -> np.ndarray:
    """layout.py:19-31: int64 global positions of ``rank``'s local tokens."""
    if not 0 <= rank < pcp_size:
        raise ValueError("rank out of range")
    if total_len % (pcp_size * interleave_size):
        raise ValueError("total_len must divide evenly across striped ranks")
    rounds = total_len // (pcp_size * interleave_size)
    starts = (np.arange(rounds, dtype=np.int64) * pcp_size + rank) * interleave_size
    return (starts[:, None] + np.arange(interleave_size, dtype=np.int64)[None, :]).reshape(-1)


def shard_query(q: np.ndarray, shape: OracleShape) -> list[np.ndarray]:
    """layout.py:34-51: per-rank ``[Hq, local_q, D]`` gathers of ``[Hq, Q, D]``."""
    return [
        q[:, global_positions(shape.current_len, r, shape.pcp_size, shape.interleave_size), :]
        for r in range(shape.pcp_size)
    ]


def shard_history(x: np.ndarray, shape: OracleShape, history_len: int) -> list[np.ndarray]:
    """layout.py:54-98: per-rank ``[blocks, Hkv, blk, D]`` caches, zero padded."""
    hkv, length, d = x.shape
    assert length == history_len
    local = history_len // shape.pcp_size
    blocks = ceil(local / shape.block_size)
    out = []
    for r in range(shape.pcp_size):
        cache = np.zeros((hkv, blocks * shape.block_size, d), dtype=x.dtype)
        cache[:, :local] = x[:, global_positions(history_len, r, shape.pcp_size, shape.interleave_size)]
        out.append(cache.reshape(hkv, blocks, shape.block_size, d).transpose(1, 0, 2, 3).copy())
    return out


def gather_history(shards: list[np.ndarray], shape: OracleShape, history_len: int) -> np.ndarray:
    """layout.py:101-132: inverse of ``shard_history``."""
    blocks, hkv, blk, d = shards[0].shape
    local = history_len // shape.pcp_size
    out = np.empty((hkv, history_len, d), dtype=shards[0].dtype)
    for r, shard in enumerate(shards):
        tokens = shard.transpose(1, 0, 2, 3).reshape(hkv, blocks * blk, d)[:, :local]
        out[:, global_positions(history_len, r, shape.pcp_size, shape.interleave_size)] = tokens
    return out


def pack_local_kv(k: np.ndarray, v: np.ndarray) -> np.ndarray:
    """kernel.py:17-29: row b = all K of block b followed by all V of block b."""
    blocks = k.shape[0]
    return np.concatenate([k.reshape(blocks, -1), v.reshape(blocks, -1)], axis=1)


def block_valid_mask(shape: OracleShape) -> np.ndarray:
    """run_poc.py:137-153: 0 / -9984 bias ``[max_local_blocks, blk/128, 1, 128]``."""
    mask = np.full((shape.max_local_blocks, shape.block_size), -9984.0, dtype=np.float32)
    remaining = shape.actual_local_history_len
    for b in range(shape.actual_local_blocks):
        valid = min(shape.block_size, remaining)
        mask[b, :valid] = 0.0
        remaining -= valid
    return mask.reshape(shape.max_local_blocks, shape.block_size // 128, 1, 128)


def page_valid_lengths(shape: OracleShape) -> np.ndarray:
    """Valid prefix of every (rank, local block): the generalised mask."""
    out = np.zeros((shape.pcp_size, shape.max_local_blocks), dtype=np.int64)
    for r in range(shape.pcp_size):
        n = shape.rank_history_len(r)
        for b in range(shape.max_local_blocks):
            out[r, b] = min(shape.block_size, max(0, n - b * shape.block_size))
    return out


# ---------------------------------------------------------------------------
# Attention (reference.py:10-95).
# ---------------------------------------------------------------------------


def kv_head_for_query_head(q_head: int, num_q_heads: int, num_kv_heads: int) -> int:
    """reference.py:10-13: Q heads are grouped contiguously per KV head."""
    return q_head // (num_q_heads // num_kv_heads)


def dense_history_attention(q: np.ndarray, k: np.ndarray, v: np.ndarray, scale: float, chunk: int = 1 << 24) -> np.ndarray:
    """reference.py:16-32 in float64: softmax(q k^T * scale) v with GQA.

    ``q`` is ``[Hq, M, D]``, ``k``/``v`` ``[Hkv, L, D]``.  Rows are processed
    in chunks of at most ``chunk`` score elements.
    """
    hq, m, d = q.shape
    hkv, length, _ = k.shape
    if hq % hkv or v.shape != k.shape or k.shape[2] != d:
        raise ValueError("incompatible Q/K/V shapes for grouped-query attention")
    group = hq // hkv
    out = np.empty((hq, m, d), dtype=np.float64)
    rows = max(1, chunk // max(length, 1))
    for g in range(hkv):
        kg = k[g].astype(np.float64)
        vg = v[g].astype(np.float64)
        qg = q[g * group:(g + 1) * group].astype(np.float64).reshape(group * m, d)
        og = np.empty_like(qg)
        for start in range(0, group * m, rows):
            s = qg[start:start + rows] @ kg.T * scale
            s -= s.max(axis=1, keepdims=True)
            np.exp(s, out=s)
            og[start:start + rows] = (s @ vg) / s.sum(axis=1, keepdims=True)
        out[g * group:(g + 1) * group] = og.reshape(group, m, d)
    return out


def expected_rows(
    q_global: np.ndarray,
    k_real: np.ndarray,
    v_real: np.ndarray,
    shape: OracleShape,
    rows: np.ndarray,
) -> np.ndarray:
    """float64 outputs of selected (rank, q_head, local token) rows.

    ``q_global`` is ``[Hq, current_len, D]``; ``k_real``/``v_real`` are the
    dequantised ``[Hkv, >= actual_history_len, D]`` history in global order.
    Only positions ``< actual_history_len`` participate.  Returns
    ``[len(rows), D]``.
    """
    length = shape.actual_history_len
    out = np.empty((len(rows), shape.head_dim), dtype=np.float64)
    positions = {}
    for i, (rank, qh, tok) in enumerate(np.asarray(rows).tolist()):
        if rank not in positions:
            positions[rank] = global_positions(shape.current_len, rank, shape.pcp_size, shape.interleave_size)
        kvh = kv_head_for_query_head(qh, shape.num_q_heads, shape.num_kv_heads)
        qrow = q_global[qh, positions[rank][tok]].astype(np.float64)[None, None, :]
        out[i] = dense_history_attention(qrow, k_real[kvh:kvh + 1, :length], v_real[kvh:kvh + 1, :length], shape.softmax_scale)[0, 0]
    return out


def expected_stacked(q_global: np.ndarray, k_real: np.ndarray, v_real: np.ndarray, shape: OracleShape) -> np.ndarray:
    """float64 ``[pcp, Hq, local_q, D]``: every rank's dense history attention."""
    length = shape.actual_history_len
    return np.stack(
        [
            dense_history_attention(qs, k_real[:, :length], v_real[:, :length], shape.softmax_scale)
            for qs in shard_query(q_global, shape)
        ]
    )


def paged_history_attention(
    q_stacked: np.ndarray,
    pool: np.ndarray,
    block_table: np.ndarray,
    valid_len: np.ndarray,
    shape: OracleShape,
    k_scale: float = 1.0,
    v_scale: float = 1.0,
) -> np.ndarray:
    """float64 model of the collapsed page loop.

    Reads every (rank, block) page through the block table, keeps its valid
    prefix (lengths clamped to [0, block_size]), and runs dense attention
    over the concatenation; ``pool`` rows are ``pack_local_kv`` payloads
    already decoded to floats.  Table entries outside ``[0, len(pool))`` are
    skipped, as the C ABI documents for the kernel (the reference's tables
    never hold such entries).
    """
    hkv, blk, d = shape.num_kv_heads, shape.block_size, shape.head_dim
    ks, vs = [], []
    for r in range(shape.pcp_size):
        for b in range(shape.max_local_blocks):
            n = min(int(valid_len[r, b]), blk)
            page_index = int(block_table[r, b])
            if n <= 0 or not 0 <= page_index < pool.shape[0]:
                continue
            page = pool[page_index].reshape(2, hkv, blk, d)
            ks.append(page[0, :, :n])
            vs.append(page[1, :, :n])
    k = np.concatenate(ks, axis=1) * k_scale
    v = np.concatenate(vs, axis=1) * v_scale
    return np.stack([dense_history_attention(q_stacked[r], k, v, shape.softmax_scale) for r in range(shape.pcp_size)])


def ring_history_attention(q_shards, k_shards, v_shards, shape: OracleShape, trace: list | None = None):
    """reference.py:35-95: every rank's two-loop ring with online softmax, FP32.

    Loop order as the reference: rank, local block, ring step (source rank
    ``(rank - step) % pcp``), Q head; FP32 ``torch.matmul``.  This is also the
    CPU baseline bench.py times.  ``trace`` (optional list) records the
    visited ``(rank, block, source_rank)`` triples.
    """
    import torch

    outputs = []
    local_len = shape.actual_local_history_len
    for rank, q in enumerate(q_shards):
        qf = q.float()
        m = torch.full((shape.num_q_heads, shape.local_q_len, 1), float("-inf"))
        l = torch.zeros_like(m)
        acc = torch.zeros_like(qf)
        for block in range(shape.actual_local_blocks):
            valid = min(shape.block_size, local_len - block * shape.block_size)
            for step in range(shape.pcp_size):
                src = (rank - step) % shape.pcp_size
                if trace is not None:
                    trace.append((rank, block, src))
                kb = k_shards[src][block, :, :valid, :].float()
                vb = v_shards[src][block, :, :valid, :].float()
                for qh in range(shape.num_q_heads):
                    kvh = kv_head_for_query_head(qh, shape.num_q_heads, shape.num_kv_heads)
                    s = torch.matmul(qf[qh], kb[kvh].transpose(0, 1)) * shape.softmax_scale
                    m_new = torch.maximum(m[qh], s.amax(dim=-1, keepdim=True))
                    rescale = torch.exp(m[qh] - m_new)
                    p = torch.exp(s - m_new)
                    acc[qh] = acc[qh] * rescale + torch.matmul(p, vb[kvh])
                    l[qh] = l[qh] * rescale + p.sum(dim=-1, keepdim=True)
                    m[qh] = m_new
        outputs.append(acc / l)
    return outputs


def attention_with_lse(
    q: np.ndarray, k: np.ndarray, v: np.ndarray, scale: float, key_limit: np.ndarray | None = None
) -> tuple[np.ndarray, np.ndarray]:
    """float64 GQA attention (reference.py:16-32) plus each row's log-sum-exp.

    ``q`` ``[Hq, M, D]``, ``k``/``v`` ``[Hkv, L, D]``; ``key_limit``
    (optional, ``[M]``) lets query row i see keys ``[0, key_limit[i])`` only
    (every head alike).  Returns ``out [Hq, M, D]`` and
    ``lse [Hq, M] = ln sum_k exp(score_k)``; a row with no key gets a zero
    output and ``-inf``.
    """
    hq, m, d = q.shape
    hkv, length, _ = k.shape
    if hq % hkv or v.shape != k.shape or k.shape[2] != d:
        raise ValueError("incompatible Q/K/V shapes for grouped-query attention")
    group = hq // hkv
    out = np.zeros((hq, m, d), dtype=np.float64)
    lse = np.full((hq, m), -np.inf, dtype=np.float64)
    visible = None
    if key_limit is not None:
        visible = np.arange(length)[None, :] < np.asarray(key_limit, dtype=np.int64)[:, None]
    for g in range(hkv):
        kg = k[g].astype(np.float64)
        vg = v[g].astype(np.float64)
        for qh in range(g * group, (g + 1) * group):
            s = q[qh].astype(np.float64) @ kg.T * scale
            if visible is not None:
                s = np.where(visible, s, -np.inf)
            mx = s.max(axis=1, keepdims=True)
            has = np.isfinite(mx[:, 0])
            mx = np.where(np.isfinite(mx), mx, 0.0)
            e = np.exp(s - mx)
            total = e.sum(axis=1)
            out[qh, has] = (e @ vg)[has] / total[has, None]
            lse[qh, has] = mx[has, 0] + np.log(total[has])
    return out, lse


def current_positions(shape: OracleShape) -> np.ndarray:
    """``[pcp, local_q]`` global current position of each rank's local token (layout.py:19-31)."""
    return np.stack(
        [global_positions(shape.current_len, r, shape.pcp_size, shape.interleave_size) for r in range(shape.pcp_size)]
    )


def expected_with_current(
    q_global: np.ndarray,
    k_cur: np.ndarray,
    v_cur: np.ndarray,
    shape: OracleShape,
    k_hist: np.ndarray | None = None,
    v_hist: np.ndarray | None = None,
) -> tuple[np.ndarray, np.ndarray]:
    """float64 ``(out, lse)`` ``[pcp, Hq, local_q, (D)]`` with current-token causal attention.

    The query at global current position g sees the current keys ``0..g``
    (``k_cur``/``v_cur`` ``[Hkv, current_len, D]`` in global order) and, when
    ``k_hist`` is given, every history key ``< actual_history_len`` too.
    """
    positions = current_positions(shape)
    length = shape.actual_history_len if k_hist is not None else 0
    if k_hist is not None:
        k = np.concatenate([k_hist[:, :length], k_cur], axis=1)
        v = np.concatenate([v_hist[:, :length], v_cur], axis=1)
    else:
        k, v = k_cur, v_cur
    outs, lses = [], []
    for r, qs in enumerate(shard_query(q_global, shape)):
        o, l = attention_with_lse(qs, k, v, shape.softmax_scale, key_limit=length + positions[r] + 1)
        outs.append(o)
        lses.append(l)
    return np.stack(outs), np.stack(lses)


def max_abs_and_mean_abs(actual: np.ndarray, expected: np.ndarray) -> tuple[float, float]:
    diff = np.abs(np.asarray(actual, dtype=np.float64) - np.asarray(expected, dtype=np.float64))
    return float(diff.max()), float(diff.mean())
