"""Pins of the e4m3 numerical model (oracle/e4m3_model.py) on the CPU.

The model is the yardstick for the e4m3-MFMA kernels' own rounding error, so
it is pinned independently of them: with its two roundings switched off it
is the float64 attention of the oracle; a scalar per-row loop written here
from the kernels' description gives the same numbers; closed forms hold
(identical keys, one dominant key, the linear-mantissa code); and its e4m3
rounding agrees with torch's float8_e4m3fn cast.
"""

from __future__ import annotations

import math

import numpy as np
import pytest
import torch

from aws_training_study_amd.pcp_attention.config import PCPAttentionConfig
from aws_training_study_amd.pcp_attention.workloads import build_paged_problem
from oracle import e4m3_model as em
from oracle import pcp_oracle as orc


def _problem(seed=3, **kw):
    base = dict(pcp_size=2, current_len=128, max_history_len=1024, actual_history_len=1000, block_size=128,
                interleave_size=32, num_q_heads=4, num_kv_heads=2, head_dim=64, backend="hip")
    base.update(kw)
    cfg = PCPAttentionConfig(**base).validate()
    return cfg, build_paged_problem(cfg, seed, kv_scale="per_tensor")


def _inputs(problem):
    qbits = problem.q_stacked.view(torch.int16).numpy().view(np.uint16)
    pool = problem.kv_pages.view(torch.uint8).numpy()
    return qbits, pool, problem.block_table.numpy(), problem.page_valid_len.numpy()


def _model(cfg, problem, **kw):
    qbits, pool, table, lens = _inputs(problem)
    return em.emulate_rows(qbits, pool, table, lens, num_kv_heads=cfg.num_kv_heads, block_size=cfg.block_size,
                           softmax_scale=cfg.softmax_scale, k_scale=problem.k_scale, v_scale=problem.v_scale, **kw)


def test_round_e4m3_matches_torch_cast():
    rng = np.random.default_rng(0)
    x = np.concatenate([rng.standard_normal(20000) * np.exp2(rng.integers(-12, 9, 20000)),
                        [0.0, -0.0, 448.0, 448.01, -463.9, 2.0 ** -9, 2.0 ** -10, 3 * 2.0 ** -10, 1.0625, 1.1875]])
    x = x[np.abs(x) < 464].astype(np.float32)
    want = torch.from_numpy(x).to(torch.float8_e4m3fn).float().numpy().astype(np.float64)
    np.testing.assert_array_equal(em.round_e4m3(x), want)


def test_fast_code_is_the_linear_interpolation_of_exp2():
    x = np.linspace(-7.0, 8.4, 4001)
    codes = em.fast_exp2_code(x)
    got = orc.decode_e4m3fn(codes)
    n = np.floor(x)
    linear = np.exp2(n) * (1 + (x - n))
    # the code is the linear form rounded to e4m3's 3 mantissa bits (normal range)
    normal = x >= -6
    np.testing.assert_allclose(got[normal], em.round_e4m3(linear[normal]), rtol=0, atol=0)
    assert np.all(np.abs(got[normal] / np.exp2(x[normal]) - 1) <= 0.125)


@pytest.mark.parametrize("kernel,head_dim", [("overlap", 256), ("tile", 64), ("tile", 128)])
def test_without_rounding_it_is_float64_attention(kernel, head_dim):
    cfg, problem = _problem(head_dim=head_dim)
    out, lse = _model(cfg, problem, kernel=kernel, q_round=False, p_round=False)
    qbits, pool, table, lens = _inputs(problem)
    shape = orc.OracleShape.from_config(cfg)
    want = orc.paged_history_attention(orc.decode_bfloat16(qbits), orc.decode_e4m3fn(pool), table, lens, shape,
                                       problem.k_scale, problem.v_scale)
    # (scores are rounded to fp32, as the MFMAs accumulate them)
    np.testing.assert_allclose(out, want, rtol=0, atol=2e-6)
    # the log-sum-exp against a direct sum over the same keys
    q = orc.decode_bfloat16(qbits)[0, 0, 0]
    k = orc.decode_e4m3fn(pool).reshape(-1, 2, cfg.num_kv_heads, cfg.block_size, head_dim)
    keys = np.concatenate([k[table[r, b], 0, 0, :lens[r, b]] for r in range(cfg.pcp_size)
                           for b in range(cfg.max_local_blocks) if lens[r, b] > 0]) * problem.k_scale
    direct = math.log(math.fsum(np.exp(keys @ q * cfg.softmax_scale)))
    assert abs(lse[0, 0, 0] - direct) < 1e-5


def _scalar_row(q_bits_row, keys, vals, tiles, c_factor, kernel, exp2):
    """One row of a kernel's arithmetic written as a plain loop: the overlap
    kernel's reference trails the tile maximum by 2.5 from a -1e30 floor;
    the tile kernel's starts at -inf and jumps to the tile maximum when that
    exceeds it by more than 2.5."""
    q = orc.decode_bfloat16(q_bits_row).astype(np.float32)
    amax = np.float32(np.abs(q).max())
    inv = np.float32(448.0) / amax
    sigma = amax / np.float32(448.0)
    q8 = np.array([em.round_e4m3(np.float32(x * inv)) for x in q])
    c = np.float32(sigma * c_factor)
    m = np.float32(-1.0e30) if kernel == "overlap" else np.float32(-np.inf)
    o = np.zeros(vals.shape[1])
    l = 0.0
    key = 0
    for n in tiles:
        s = [np.float32(float(np.dot(q8, keys[key + i]))) for i in range(n)]
        mxs = np.float32(np.float32(max(s)) * c)
        if kernel == "overlap":
            m_new = max(m, np.float32(mxs - np.float32(2.5)))
        else:
            m_new = mxs if mxs > np.float32(m + np.float32(2.5)) else m
        alpha = 2.0 ** float(np.float32(m - m_new)) if m_new != m else 1.0
        m = m_new
        o *= alpha
        l *= alpha
        for i in range(n):
            if exp2 == "fast":
                y = np.float32(float(s[i]) * float(np.float32(8) * c) + float(np.float32(-8.0 * float(m) + 104.0)))
                p = float(orc.decode_e4m3fn(np.uint8(min(255, max(0, int(np.rint(float(y))))))))
            else:
                x = np.float32(float(s[i]) * float(c) + float(np.float32(6.0 - float(m))))
                p = float(em.round_e4m3(np.float32(2.0 ** float(x))))
            o += p * vals[key + i]
            l += p
        key += n
    return o / l


@pytest.mark.parametrize("kernel,exp2", [("overlap", "fast"), ("overlap", "exact"), ("tile", "exact")])
def test_vectorised_model_equals_a_scalar_loop(kernel, exp2):
    cfg, problem = _problem(head_dim=256 if kernel == "overlap" else 128, actual_history_len=777, seed=9)
    rows = np.array([[0, 0, 0], [1, 3, 63], [0, 2, 17]])
    out, _ = _model(cfg, problem, kernel=kernel, exp2=exp2, rows=rows)
    qbits, pool, table, lens = _inputs(problem)
    walk = em.walk_pages(table, lens, pool.shape[0], cfg.block_size)
    tiles = em._tiles(walk)
    dec = orc.decode_e4m3fn(pool).reshape(-1, 2, cfg.num_kv_heads, cfg.block_size, cfg.head_dim)
    c_factor = np.float32(np.float32(np.float32(cfg.softmax_scale) * np.float32(problem.k_scale)) * em.LOG2E)
    group = cfg.num_q_heads // cfg.num_kv_heads
    for i, (rank, qh, tok) in enumerate(rows):
        g = qh // group
        keys = np.concatenate([dec[p, 0, g, b:b + n] for p, b, n in tiles])
        vals = np.concatenate([dec[p, 1, g, b:b + n] for p, b, n in tiles])
        want = _scalar_row(qbits[rank, qh, tok], keys, vals, [n for _, _, n in tiles], c_factor, kernel, exp2)
        np.testing.assert_allclose(out[i], want * problem.v_scale, rtol=1e-12, atol=1e-12)


@pytest.mark.parametrize("kernel,exp2", [("overlap", "fast"), ("overlap", "exact"), ("tile", "exact")])
def test_identical_keys_give_the_mean_of_v(kernel, exp2):
    """Equal scores give equal probabilities whatever their rounding: O = mean(V)."""
    cfg, problem = _problem(head_dim=256 if kernel == "overlap" else 128, actual_history_len=1024)
    pool = problem.kv_pages.view(torch.uint8).numpy().copy().reshape(-1, 2, cfg.num_kv_heads, cfg.block_size,
                                                                     cfg.head_dim)
    pool[:, 0] = pool[0, 0, :, :1]  # every key of every page equals one key
    qbits, _, table, lens = _inputs(problem)
    out, _ = em.emulate_rows(qbits, pool.reshape(pool.shape[0], -1), table, lens, num_kv_heads=cfg.num_kv_heads,
                             block_size=cfg.block_size, softmax_scale=cfg.softmax_scale, k_scale=problem.k_scale,
                             v_scale=problem.v_scale, kernel=kernel, exp2=exp2)
    dec = orc.decode_e4m3fn(pool)
    mean_v = np.stack([np.concatenate([dec[table[r, b], 1, g, :lens[r, b]] for r in range(cfg.pcp_size)
                                       for b in range(cfg.max_local_blocks)]).mean(0) for g in range(2)])
    group = cfg.num_q_heads // cfg.num_kv_heads
    want = np.stack([mean_v[h // group] for h in range(cfg.num_q_heads)])[None, :, None, :] * problem.v_scale
    np.testing.assert_allclose(out, np.broadcast_to(want, out.shape), rtol=1e-12, atol=1e-12)


def test_a_dominant_key_gives_its_value():
    cfg, problem = _problem(head_dim=256, actual_history_len=512, seed=4)
    qbits, pool, table, lens = _inputs(problem)
    dec = pool.reshape(-1, 2, cfg.num_kv_heads, cfg.block_size, cfg.head_dim).copy()
    # key 5 of page table[0, 0] aligned with row (0, 0, 0)'s query, scaled far above the rest
    q = orc.decode_bfloat16(qbits[0, 0, 0])
    code = torch.from_numpy((np.sign(q) * 448).astype(np.float32)).to(torch.float8_e4m3fn).view(torch.uint8).numpy()
    dec[table[0, 0], 0, 0, 5] = code
    out, _ = em.emulate_rows(qbits, dec.reshape(dec.shape[0], -1), table, lens, num_kv_heads=cfg.num_kv_heads,
                             block_size=cfg.block_size, softmax_scale=cfg.softmax_scale, k_scale=problem.k_scale,
                             v_scale=problem.v_scale, kernel="overlap", rows=np.array([[0, 0, 0]]))
    v = orc.decode_e4m3fn(dec[table[0, 0], 1, 0, 5]) * problem.v_scale
    np.testing.assert_allclose(out[0], v, rtol=0, atol=1e-9)


def test_splits_merge_to_the_one_pass_result_without_rounding():
    cfg, problem = _problem(head_dim=256, actual_history_len=1000)
    one, lse1 = _model(cfg, problem, kernel="overlap", q_round=False, p_round=False)
    three, lse3 = _model(cfg, problem, kernel="overlap", q_round=False, p_round=False, splits=3)
    # (the fp32 exponent arguments round differently against other references)
    np.testing.assert_allclose(three, one, rtol=0, atol=1e-6)
    np.testing.assert_allclose(lse3, lse1, rtol=0, atol=1e-6)


def test_mass_is_the_probability_sum_against_the_reference():
    """mass = sum_k 2^(x_k - m) with m within 2.5 of the largest x_k; split
    masses recombine against the largest range reference."""
    cfg, problem = _problem(head_dim=256, actual_history_len=1000)
    rows = np.array([[0, 1, 5], [1, 2, 60]])
    _, lse, mass = _model(cfg, problem, kernel="overlap", exp2="exact", rows=rows, return_mass=True)
    qbits, pool, table, lens = _inputs(problem)
    shape = orc.OracleShape.from_config(cfg)
    # natural-log sum of exp(score) over all keys vs log2 mass: mass * 2^m = sum 2^x
    _, lse_plain = _model(cfg, problem, kernel="overlap", q_round=False, p_round=False, rows=rows)
    for i in range(len(rows)):
        # the largest probability (2^(x_max - m) in [1, 2^2.5]) bounds the mass from below
        assert mass[i] >= 1.0
    _, _, mass3 = _model(cfg, problem, kernel="overlap", exp2="exact", rows=rows, return_mass=True, splits=3)
    np.testing.assert_allclose(mass3, mass, rtol=0.3)  # the same keys, rounded against other references
    assert shape.head_dim == 256 and np.all(np.isfinite(lse_plain))


# ---- the guard's threshold and the spread of V


def _pool_with_v(cfg, v_codes_fn):
    """A zero pool of cfg's shape whose V codes come from v_codes_fn(page, head) -> [block, D] float (e4m3 values)."""
    pages = cfg.pcp_size * cfg.max_local_blocks
    pool = np.zeros((pages, 2, cfg.num_kv_heads, cfg.block_size, cfg.head_dim), dtype=np.float32)
    for page in range(pages):
        for h in range(cfg.num_kv_heads):
            pool[page, 1, h] = v_codes_fn(page, h)
    codes = torch.from_numpy(pool).to(torch.float8_e4m3fn).view(torch.uint8).numpy()
    table = np.arange(pages, dtype=np.int32).reshape(cfg.pcp_size, cfg.max_local_blocks)
    lens = np.full(table.shape, cfg.block_size, dtype=np.int32)
    return codes.reshape(pages, -1), table, lens


def test_guard_threshold_closed_forms():
    """Identical V rows have no spread: threshold 0.  V codes +a_d / -a_d on
    alternate keys have variance a_d^2 in channel d: 384 v_scale^2 max_d
    a_d^2.  The threshold scales with v_scale^2 and ignores a common offset."""
    cfg = PCPAttentionConfig(pcp_size=2, current_len=128, max_history_len=1024, actual_history_len=1024,
                             block_size=128, interleave_size=32, num_q_heads=4, num_kv_heads=2, head_dim=64,
                             backend="hip").validate()
    kw = dict(num_kv_heads=2, block_size=128, head_dim=64)
    row = np.linspace(-3, 3, 64).astype(np.float32)
    same = _pool_with_v(cfg, lambda page, h: np.broadcast_to(row, (128, 64)))
    np.testing.assert_array_equal(em.guard_thresholds(*same, v_scale=0.7, **kw), [0.0, 0.0])
    amp = np.array([0.5, 2.0])  # head 0: channels at +-0.5 .. , head 1: up to +-2 in channel 63
    sign = np.where(np.arange(128) % 2 == 0, 1.0, -1.0)[:, None]

    def two_point(page, h):
        a_d = np.full(64, 0.25, dtype=np.float32)
        a_d[63] = amp[h]
        return (sign * a_d).astype(np.float32)
    pool = _pool_with_v(cfg, two_point)
    np.testing.assert_allclose(em.guard_thresholds(*pool, v_scale=1.0, **kw), 384 * amp ** 2, rtol=1e-12)
    np.testing.assert_allclose(em.guard_thresholds(*pool, v_scale=0.5, **kw), 384 * 0.25 * amp ** 2, rtol=1e-12)
    shifted = _pool_with_v(cfg, lambda page, h: two_point(page, h) + 3.0)
    np.testing.assert_allclose(em.guard_thresholds(*shifted, v_scale=1.0, **kw), 384 * amp ** 2, rtol=1e-12)


def test_guard_threshold_samples_every_s_th_key_of_long_walks():
    """Beyond 2048 valid keys the statistics take every s-th key of each
    page (s a power of two): keys off the stride do not count."""
    cfg = PCPAttentionConfig(pcp_size=4, current_len=256, max_history_len=32768, actual_history_len=32768,
                             block_size=512, interleave_size=64, num_q_heads=4, num_kv_heads=1, head_dim=64,
                             backend="hip").validate()
    keys = np.arange(512)[:, None]
    # on the stride (16: 32768 keys / 16 = 2048) alternate +-1; off it 448
    v = np.where(keys % 16 == 0, np.where((keys // 16) % 2 == 0, 1.0, -1.0), 448.0)
    pool = _pool_with_v(cfg, lambda page, h: np.broadcast_to(v, (512, 64)).astype(np.float32))
    kw = dict(num_kv_heads=1, block_size=512, head_dim=64)
    np.testing.assert_allclose(em.guard_thresholds(*pool, v_scale=1.0, **kw), [384.0], rtol=1e-12)
    # half the history: 16384 keys, every eighth one (448 among them)
    lens = pool[2].copy()
    lens[:, cfg.max_local_blocks // 2:] = 0
    full = em.guard_thresholds(pool[0], pool[1], lens, v_scale=1.0, **kw)
    assert full[0] > 384 * 1e4


def test_guard_threshold_keeps_wide_v_rows_within_half_the_bar():
    """The e4m3 rounding error of a row grows with the spread of V.  With V ~
    N(0, 16) over 2048 keys the rows a fixed mass threshold of 384 would
    keep on e4m3 MFMAs reach 2e-2; the threshold 384 * v_scale^2 * max_d
    Var(V) keeps rows within about half the bar whatever the spread (V ~
    N(0, 1) and N(0, 16) over 2048 keys, N(0, 4) over 8192 keys, where most
    rows are kept), as unit-variance V does at 384.  Error: the model
    against itself with both roundings off."""
    rng = np.random.default_rng(5)
    rows = np.stack([rng.integers(0, 4, 64), rng.integers(0, 8, 64), rng.integers(0, 64, 64)], axis=1)

    def case(tokens, v_factor):
        cfg = PCPAttentionConfig(pcp_size=4, current_len=256, max_history_len=tokens, actual_history_len=tokens,
                                 block_size=256, interleave_size=64, num_q_heads=8, num_kv_heads=2, head_dim=256,
                                 backend="hip").validate()
        problem = build_paged_problem(cfg, 7, kv_scale="per_tensor", v_factor=v_factor)
        qbits, pool, table, lens = _inputs(problem)
        kw = dict(num_kv_heads=2, block_size=256, softmax_scale=cfg.softmax_scale, k_scale=problem.k_scale,
                  v_scale=problem.v_scale, rows=rows)
        got, _, mass = em.emulate_rows(qbits, pool, table, lens, return_mass=True, **kw)
        exact, _ = em.emulate_rows(qbits, pool, table, lens, q_round=False, p_round=False, **kw)
        thr = em.guard_thresholds(pool, table, lens, num_kv_heads=2, block_size=256, head_dim=256,
                                  v_scale=problem.v_scale)[rows[:, 1] // 4]
        return np.abs(got - exact).max(axis=1), mass, thr

    err, mass, thr = case(2048, 1.0)
    assert 350 < thr.max() < 450 and (mass >= thr).sum() >= 8
    assert err[mass >= thr].max() <= 1.2e-2
    err, mass, thr = case(2048, 4.0)
    assert 14 * 384 < thr.min() < 19 * 384
    assert err[mass >= 384].max() > 2e-2          # what the fixed threshold would keep
    assert err[mass >= thr].max(initial=0.0) <= 1.2e-2
    err, mass, thr = case(8192, 2.0)
    assert (mass >= thr).sum() >= 32
    assert err[mass >= thr].max() <= 1.2e-2
