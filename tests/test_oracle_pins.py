"""Pins of the CPU oracle (oracle/reference_cpu.py) — CPU only.

The reference commits no golden tensors; its check_math.py is the known-answer
suite. Each oracle function is pinned here by something other than its own
formula: check_math.py's independent references (restated as such), token-level
brute force on tiny shapes, closed forms / known answers, and invariants, chosen
so a plausible mistake (wrong divisor, off-by-one validity rule, missing ln n,
wrong softmax axis, transposed operand) fails at least one of them.
"""

import itertools
import math

import numpy as np
import pytest
import torch

from oracle import reference_cpu as ref

SCALE = 128 ** -0.5


def rnd(shape, seed, scale=1.0):
    rng = np.random.default_rng(seed)
    return ref.bf16_round((rng.standard_normal(shape) * scale).astype(np.float32))


# ------------------------------------------------------------------ bf16

def test_bf16_round_matches_torch():
    rng = np.random.default_rng(0)
    x = np.concatenate([
        rng.standard_normal(10000).astype(np.float32) * 10.0 ** rng.integers(-30, 30, 10000),
        np.array([0.0, -0.0, np.inf, -np.inf, 1.0 + 2 ** -8, 1.0 + 3 * 2 ** -8, 3e-39, -1e-40,
                  65504.0, 3.4e38], np.float32),
    ]).astype(np.float32)
    expected = torch.from_numpy(x).to(torch.bfloat16).float().numpy()
    np.testing.assert_array_equal(ref.bf16_round(x), expected)
    assert np.isnan(ref.bf16_round(np.array([np.nan], np.float32)))[0]


# --------------------------------------------------------------- pooling

def test_block_mean_k_against_loop_and_known_answers():
    k = rnd((2, 300, 3, 8), 1)
    got = ref.block_mean_k(k)
    for b, j, h in itertools.product(range(2), range(3), range(3)):
        rows = k[b, j * 128:min(300, j * 128 + 128), h]
        for d in range(8):
            total = np.float32(math.fsum(float(x) for x in rows[:, d]))
            want = ref.bf16_round(np.array([total / np.float32(len(rows))], np.float32))[0]
            assert got[b, j, h, d] == want
    # partial last block divides by its valid count, not the block size
    k = np.zeros((1, 130, 1, 2), np.float32)
    k[0, 128:, 0, :] = 0.75
    assert ref.block_mean_k(k)[0, 1, 0, 0] == 0.75
    k = np.full((1, 5, 1, 1), 0.5, np.float32)
    assert ref.block_mean_k(k)[0, 0, 0, 0] == 0.5


def test_block_descriptors_against_two_pass_and_known_answers():
    k = rnd((1, 300, 2, 8), 2)
    v = rnd((1, 300, 2, 8), 3)
    d = ref.block_descriptors(k, v)
    for j in range(3):
        sl = slice(j * 128, min(300, j * 128 + 128))
        np.testing.assert_allclose(d.mean_k[0, j], k[0, sl].astype(np.float64).mean(0), atol=1e-6)
        np.testing.assert_allclose(d.var_k[0, j], k[0, sl].astype(np.float64).var(0), atol=2e-5)
        np.testing.assert_allclose(d.mean_v[0, j], v[0, sl].astype(np.float64).mean(0), atol=1e-6)
        np.testing.assert_allclose(d.sigma_v[0, j],
                                   np.sqrt(v[0, sl].astype(np.float64).var(0).sum(-1)), atol=2e-5)
    np.testing.assert_array_equal(d.counts, [128, 128, 44])
    # alternating +-a: mean 0, variance a^2, sigma_v = a sqrt(D)
    a = 1.5
    x = np.zeros((1, 128, 1, 4), np.float32)
    x[0, ::2] = a
    x[0, 1::2] = -a
    dd = ref.block_descriptors(x, x)
    assert (dd.mean_k == 0).all() and np.allclose(dd.var_k, a * a)
    assert np.isclose(dd.sigma_v[0, 0, 0], a * 2.0)
    # constant block: one-pass variance is clamped at 0, never negative
    c = np.full((1, 77, 1, 4), 0.3, np.float32)
    assert (ref.block_descriptors(c, c).var_k >= 0).all()


# ---------------------------------------------------------- V1 scores

def check_math_v1_score_reference(q, mean_k, scale, block_size=128):
    """check_math.py:45-61 (joint max over rows and blocks, natural exp)."""
    batch, sequence, heads, _ = q.shape
    blocks = mean_k.shape[1]
    kk = np.repeat(mean_k, heads // mean_k.shape[2], axis=2).astype(np.float64)
    logits = np.einsum("bqhd,bkhd->bhqk", q.astype(np.float64), kk) * scale
    key_ends = (np.arange(blocks) + 1) * block_size - 1
    logits = np.where(np.arange(sequence)[:, None] < key_ends[None, :], -np.inf, logits)
    pad = blocks * block_size - sequence
    logits = np.concatenate([logits, np.full((batch, heads, pad, blocks), -np.inf)], axis=2)
    logits = logits.reshape(batch, heads, blocks, block_size, blocks)
    maximum = logits.max(axis=(3, 4), keepdims=True)
    maximum = np.where(np.isfinite(maximum), maximum, 0.0)
    mass = np.exp(logits - maximum).sum(axis=3)
    normalized = mass / (mass.sum(axis=-1, keepdims=True) + 1e-9)
    return normalized.transpose(0, 2, 3, 1)


@pytest.mark.parametrize("length", (257, 1089))
def test_v1_scores_against_check_math_reference(length):
    q = rnd((1, length, 4, 128), 4)
    k = rnd((1, length, 2, 128), 5)
    kbar = ref.block_mean_k(k)
    got = ref.v1_scores(q, kbar, SCALE)
    want = check_math_v1_score_reference(q, kbar, SCALE)
    np.testing.assert_allclose(got, want, atol=1e-6, rtol=1e-5)
    rows = got.sum(axis=2)
    assert np.all(np.isclose(rows, 1.0, atol=1e-5) | (rows == 0))
    upper = np.triu(np.ones(got.shape[1:3], bool), 1)
    assert (got[:, upper] == 0).all()


@pytest.mark.parametrize("length", (1, 100, 127))
def test_v1_scores_without_valid_rows_are_zero(length):
    """normalize_scores' ``+ 1e-9`` (upstream :410-417): a sequence shorter than
    one block has no valid row for any key block (rows i >= 127 only), so every
    weight is 0 and the score is 0 / (0 + 1e-9) = 0, not 0 / 0."""
    q = rnd((1, length, 2, 16), 8)
    kbar = ref.block_mean_k(rnd((1, length, 1, 16), 9))
    mass, maximum = ref.v1_scores_raw(q, kbar, SCALE)
    assert (maximum == -np.inf).all() and (mass == 0).all()
    got = ref.v1_scores(q, kbar, SCALE)
    assert np.isfinite(got).all() and (got == 0).all()
    # the same for a row of the normaliser fed directly: no finite maximum
    direct = ref.normalize_scores(np.zeros((1, 2, 2, 1), np.float32),
                                  np.full((1, 2, 2, 1), -np.inf, np.float32))
    assert np.isfinite(direct).all() and (direct == 0).all()


def test_v1_raw_diagonal_uses_last_row_only():
    q = rnd((1, 300, 2, 16), 6)
    kbar = ref.block_mean_k(rnd((1, 300, 1, 16), 7))
    mass, maximum = ref.v1_scores_raw(q, kbar, SCALE)
    c = np.float32(SCALE * ref.LOG2E)
    for t in range(2):
        row = (t + 1) * 128 - 1
        for h in range(2):
            x = np.float32(np.float32(q[0, row, h].astype(np.float64) @ kbar[0, t, 0]) * c)
            assert maximum[0, t, t, h] == x and mass[0, t, t, h] == 1.0
    # last tile holds rows 256..299 < 383: no valid row on its diagonal
    assert (maximum[0, 2, 2] == -np.inf).all() and (mass[0, 2, 2] == 0).all()


def test_v1_scores_brute_force_tiny():
    length, bs = 11, 4
    q = rnd((1, length, 2, 3), 8)
    kbar = ref.bf16_round(rnd((1, 3, 1, 3), 9))
    got = ref.v1_scores(q, kbar, 0.7, block_size=bs)
    blocks = 3
    for t, h in itertools.product(range(blocks), range(2)):
        weights = []
        for j in range(blocks):
            xs = [float(np.float32(np.float32(sum(float(q[0, i, h, d]) * float(kbar[0, j, 0, d])
                                                  for d in range(3))) * np.float32(0.7 * ref.LOG2E)))
                  for i in range(t * bs, min(length, t * bs + bs)) if i >= (j + 1) * bs - 1]
            weights.append((max(xs), sum(2.0 ** (x - max(xs)) for x in xs)) if xs else None)
        finite = [w for w in weights if w is not None]
        g = max(w[0] for w in finite) if finite else 0.0
        w = [0.0 if x is None else x[1] * 2.0 ** (x[0] - g) for x in weights]
        total = sum(w) + 1e-9
        for j in range(blocks):
            assert got[0, t, j, h] == pytest.approx(w[j] / total, rel=1e-5, abs=1e-7)


# ----------------------------------------------------------- selection

def brute_select(scores, sink, window, alpha, last, min_budget=0, positive=False, zero_alpha_causal=False):
    b_, qb, kb, hh = scores.shape
    active = np.zeros(scores.shape, bool)
    for b, t, h in itertools.product(range(b_), range(qb), range(hh)):
        row = [float(scores[b, t, j, h]) for j in range(kb)]
        mx = max(row)
        thr = float(np.float32(np.float32(mx) * np.float32(alpha)))
        order = sorted(range(kb), key=lambda j: (-row[j], j))[:min_budget]
        for j in range(kb):
            if zero_alpha_causal and alpha == 0:
                keep = True
            else:
                keep = row[j] >= thr and (row[j] > 0 or not positive)
            keep = keep or j in order
            prot = j < sink or 0 <= t - j < window or t >= qb - last
            active[b, t, j, h] = (keep or prot) and j <= t
    return active


@pytest.mark.parametrize("sink,window,alpha,last,budget", [
    (2, 4, 0.08, 2, 0), (0, 0, 0.5, 0, 0), (1, 1, 0.9, 1, 2), (3, 2, 0.0, 0, 0), (0, 1, 1.0, 0, 1)])
def test_deal_output_score_brute_force(sink, window, alpha, last, budget):
    rng = np.random.default_rng(10)
    scores = rng.random((2, 9, 9, 3)).astype(np.float32)
    scores[0, :, :, 0] = np.round(scores[0, :, :, 0], 1)     # plenty of exact ties
    idx, cnt = ref.deal_output_score(scores, sink, window, alpha, last, budget)
    active = brute_select(scores, sink, window, alpha, last, budget)
    np.testing.assert_array_equal(cnt, active.sum(axis=2))
    for b, t, h in itertools.product(range(2), range(9), range(3)):
        listed = [j for j in range(9) if active[b, t, j, h]]
        assert idx[b, t, :, h].tolist() == listed + [9] * (9 - len(listed))
    assert idx.dtype == np.int64 and cnt.dtype == np.int32


def test_deal_output_score_special_cases():
    scores = np.random.default_rng(11).random((1, 6, 6, 2)).astype(np.float32)
    _, cnt = ref.deal_output_score(scores, 0, 0, 0.0, 0, 0)        # alpha 0: every causal block
    np.testing.assert_array_equal(cnt[0, :, 0], np.arange(1, 7))
    _, cnt = ref.deal_output_score(scores, 0, 0, 2.0, 2, 0)        # last two tiles: all causal
    assert cnt[0, 4, 0] == 5 and cnt[0, 5, 0] == 6
    _, cnt = ref.deal_output_score(np.zeros_like(scores), 0, 0, 0.5, 0, 0)   # 0 >= 0: all kept
    np.testing.assert_array_equal(cnt[0, :, 1], np.arange(1, 7))


@pytest.mark.parametrize("alpha", (0.0, 0.08, 0.5))
def test_protected_selection_brute_force(alpha):
    rng = np.random.default_rng(12)
    scores = rng.random((1, 8, 8, 3)).astype(np.float32)
    scores[:, :, 3] = 0.0     # zero scores are never routed (only protected)
    got = ref.protected_selection(scores, alpha, 2, 1, 1)
    np.testing.assert_array_equal(got, brute_select(scores, 2, 1, alpha, 1, positive=True,
                                                    zero_alpha_causal=True))


def test_mask_index_round_trip():
    rng = np.random.default_rng(13)
    mask = rng.random((2, 7, 7, 3)) < 0.4
    idx, cnt = ref.indices_from_mask(mask)
    np.testing.assert_array_equal(ref.mask_from_indices(idx, cnt), mask)
    for b, t, h in itertools.product(range(2), range(7), range(3)):
        ids = idx[b, t, :, h]
        assert (np.diff(ids) >= 0).all() and (ids[cnt[b, t, h]:] == 7).all()


# ------------------------------------------------------- new selectors

def check_math_selector_reference(q, d, scale, selector, block=128):
    """check_math.py:165-191 (per-tile softmax over the tile's visible blocks)."""
    batch, sequence, heads, _ = q.shape
    blocks = d.mean_k.shape[1]
    group = heads // d.mean_k.shape[2]
    mk = np.repeat(d.mean_k, group, 2).astype(np.float64)
    vk = np.repeat(d.var_k, group, 2).astype(np.float64)
    sv = np.repeat(d.sigma_v, group, 2).transpose(0, 2, 1).astype(np.float64)
    out = np.zeros((batch, blocks, blocks, heads))
    for tile in range(1, blocks):
        query = q[:, tile * block:min(sequence, tile * block + block)].astype(np.float64)
        ell0 = np.einsum("bqhd,bkhd->bqhk", query, mk[:, :tile]) * scale
        ell0 += np.log(d.counts[:tile].astype(np.float64)).reshape(1, 1, 1, tile)
        if selector == "mean_balanced":
            logits, mult = ell0, 1.0
        else:
            u = np.maximum(np.einsum("bqhd,bkhd->bqhk", query ** 2, vk[:, :tile]) * scale * scale, 0)
            logits = ell0 + 0.5 * u
            mult = 1.0 if selector == "cgf_mean" else np.sqrt(u) * sv[:, None, :, :tile]
        p = np.exp(logits - logits.max(-1, keepdims=True))
        p /= p.sum(-1, keepdims=True)
        out[:, tile, :tile] = (p * mult).mean(axis=1).transpose(0, 2, 1)
    return out


@pytest.mark.parametrize("selector", ref.SELECTORS)
def test_selector_scores_against_check_math(selector):
    q = rnd((1, 300, 4, 16), 14)
    k = rnd((1, 300, 2, 16), 15)
    v = rnd((1, 300, 2, 16), 16)
    d = ref.block_descriptors(k, v)
    got = ref.selector_scores(q, d, 0.25, selector)
    np.testing.assert_allclose(got, check_math_selector_reference(q, d, 0.25, selector),
                               atol=1e-7, rtol=1e-6)
    with pytest.raises(ValueError):
        ref.selector_scores(q, d, 0.25, "bogus")


def test_selector_scores_known_answers():
    q = rnd((1, 4 * 128, 2, 8), 17)
    same = np.broadcast_to(rnd((1, 1, 1, 8), 18), (1, 4, 1, 8)).copy()
    zeros = np.zeros((1, 4, 1, 8), np.float32)
    d = ref.BlockDescriptors(same, same, zeros, np.zeros((1, 4, 1), np.float32),
                             np.full(4, 128, np.int32))
    bal = ref.selector_scores(q, d, SCALE, "mean_balanced")
    for t in range(1, 4):
        np.testing.assert_allclose(bal[0, t, :t], 1.0 / t, rtol=1e-6)     # uniform over j < t
    assert (bal[0, 0] == 0).all() and (np.triu(np.ones((4, 4)), 0)[None, :, :, None] * bal == 0).all()
    np.testing.assert_array_equal(ref.selector_scores(q, d, SCALE, "cgf_mean"), bal)   # var 0
    assert (ref.selector_scores(q, d, SCALE, "dispersion_mean") == 0).all()            # sigma 0
    # one visible block (t = 1): dispersion score = mean over rows of sqrt(u) * sigma_v
    var = np.full((1, 4, 1, 8), 0.5, np.float32)
    sig = np.full((1, 4, 1), 2.0, np.float32)
    d2 = ref.BlockDescriptors(same, same, var, sig, np.full(4, 128, np.int32))
    disp = ref.selector_scores(q, d2, SCALE, "dispersion_mean")
    u = np.maximum((q[0, 128:256, 0].astype(np.float64) ** 2 @ var[0, 0, 0]) * SCALE ** 2, 0)
    assert disp[0, 1, 0, 0] == pytest.approx((np.sqrt(u) * 2.0).mean(), rel=1e-6)


# ---------------------------------------------------- exact attention

def dense_reference(q, k, v, scale):
    """check_math.py:33-42."""
    heads = q.shape[2]
    kk = np.repeat(k, heads // k.shape[2], 2).astype(np.float64)
    vv = np.repeat(v, heads // v.shape[2], 2).astype(np.float64)
    logits = np.einsum("bqhd,bkhd->bhqk", q.astype(np.float64), kk) * scale
    pos = np.arange(q.shape[1])
    logits = np.where(pos[None, :] > pos[:, None], -np.inf, logits)
    m = logits.max(-1, keepdims=True)
    w = np.exp(logits - m)
    lse = (m[..., 0] + np.log(w.sum(-1))).transpose(0, 2, 1)
    out = np.einsum("bhqk,bkhd->bqhd", w / w.sum(-1, keepdims=True), vv)
    return out, lse


def test_exact_attention_all_selected_equals_dense():
    q, k, v = rnd((1, 300, 4, 16), 19), rnd((1, 300, 2, 16), 20), rnd((1, 300, 2, 16), 21)
    blocks = 3
    sel = np.broadcast_to(np.tril(np.ones((blocks, blocks), bool))[None, :, :, None], (1, 3, 3, 4))
    idx, cnt = ref.indices_from_mask(sel)
    out, lse = ref.exact_attention(q, k, v, idx, cnt, 0.3)
    d_out, d_lse = dense_reference(q, k, v, 0.3)
    np.testing.assert_array_equal(out, ref.bf16_round(d_out.astype(np.float32)))
    np.testing.assert_allclose(lse, d_lse, atol=1e-6)


def test_exact_attention_token_brute_force_and_edges():
    bs, length = 4, 11
    q, k, v = rnd((1, length, 2, 3), 22), rnd((1, length, 1, 3), 23), rnd((1, length, 1, 3), 24)
    idx = np.full((1, 3, 3, 2), 3, np.int64)
    cnt = np.zeros((1, 3, 2), np.int32)
    idx[0, 2, :2, 0] = [0, 2]; cnt[0, 2, 0] = 2          # skip block 1
    idx[0, 1, :1, 1] = [2]; cnt[0, 1, 1] = 1             # a future block: not causally masked
    idx[0, 2, :1, 1] = [2]; cnt[0, 2, 1] = 1             # diagonal only (row 8 sees key 8 only)
    out, lse = ref.exact_attention(q, k, v, idx, cnt, 0.5, block_size=bs)
    for i, h in itertools.product(range(length), range(2)):
        t = i // bs
        keys = []
        for j in idx[0, t, :cnt[0, t, h], h]:
            for p in range(j * bs, j * bs + bs):
                if j == t and p > i:
                    continue
                keys.append(p)
        if not keys:
            assert (out[0, i, h] == 0).all() and lse[0, i, h] == -np.inf
            continue
        kv = lambda arr, p: arr[0, p, 0].astype(np.float64) if p < length else np.zeros(3)
        lg = np.array([q[0, i, h].astype(np.float64) @ kv(k, p) for p in keys]) * 0.5
        w = np.exp(lg - lg.max())
        want = (w[:, None] * np.array([kv(v, p) for p in keys])).sum(0) / w.sum()
        np.testing.assert_array_equal(out[0, i, h], ref.bf16_round(want.astype(np.float32)))
        assert lse[0, i, h] == pytest.approx(lg.max() + np.log(w.sum()), abs=1e-6)
    # row 8 (first row of tile 2), head 1: only key 8 -> output v[8], lse = scale q.k
    np.testing.assert_array_equal(out[0, 8, 1], v[0, 8, 0])


def test_exact_attention_future_kv_invariance():
    """check_math.py:322-329 at the oracle level."""
    q, k, v = rnd((1, 257, 4, 8), 25), rnd((1, 257, 2, 8), 26), rnd((1, 257, 2, 8), 27)
    sel = ref.protected_selection(np.zeros((1, 3, 3, 4), np.float32), 0.0, 2, 4, 2)
    sel[:, 2, 1, ::2] = False
    idx, cnt = ref.indices_from_mask(sel)
    first, _ = ref.exact_attention(q, k, v, idx, cnt, SCALE)
    k2, v2 = k.copy(), v.copy()
    k2[:, 200:] *= 19
    v2[:, 200:] += 23
    second, _ = ref.exact_attention(q, k2, v2, idx, cnt, SCALE)
    np.testing.assert_array_equal(first[:, :200], second[:, :200])


# -------------------------------------------------- mean tail + merge

def explicit_mean_reference(q, k, v, selected, d, scale, block=128):
    """check_math.py:81-119 (token-level exact mask plus block-mean logits)."""
    batch, sequence, heads, _ = q.shape
    blocks = selected.shape[1]
    group = heads // k.shape[2]
    ke = np.repeat(k, group, 2).astype(np.float64)
    ve = np.repeat(v, group, 2).astype(np.float64)
    mk = np.repeat(d.mean_k, group, 2).astype(np.float64)
    mv = np.repeat(d.mean_v, group, 2).astype(np.float64)
    exact = np.einsum("bqhd,bkhd->bqhk", q.astype(np.float64), ke) * scale
    pos = np.arange(sequence)
    qt = pos // block
    rows = selected.transpose(0, 1, 3, 2)[:, qt]
    allowed = rows[:, :, :, pos // block] & (pos[None, None, None, :] <= pos[None, :, None, None])
    exact = np.where(allowed, exact, -np.inf)
    mean = np.einsum("bqhd,bkhd->bqhk", q.astype(np.float64), mk) * scale
    mean += np.log(d.counts.astype(np.float64)).reshape(1, 1, 1, blocks)
    mean_allowed = (np.arange(blocks)[None, None, None, :] < qt[None, :, None, None]) & ~rows
    mean = np.where(mean_allowed, mean, -np.inf)
    total = np.logaddexp(np.log(np.exp(exact).sum(-1)), np.log(np.exp(mean).sum(-1)))
    out = np.einsum("bqhk,bkhd->bqhd", np.exp(exact - total[..., None]), ve) + \
        np.einsum("bqhk,bkhd->bqhd", np.where(mean_allowed, np.exp(mean - total[..., None]), 0), mv)
    return out, total


def test_exact_plus_mean_against_check_math():
    q, k, v = rnd((1, 385, 4, 8), 28), rnd((1, 385, 2, 8), 29), rnd((1, 385, 2, 8), 30)
    sel = ref.protected_selection(np.zeros((1, 4, 4, 4), np.float32), 0.0, 2, 4, 2)
    sel[:, 2, 0, ::2] = False
    sel[:, 3, 1, :] = False
    d = ref.block_descriptors(k, v)
    idx, cnt = ref.indices_from_mask(sel)
    merged, total = ref.merge_exact_mean(*ref.exact_attention(q, k, v, idx, cnt, SCALE),
                                         *ref.mean_tail(q, d, sel, SCALE))
    want, want_total = explicit_mean_reference(q, k, v, sel, d, SCALE)
    np.testing.assert_allclose(merged, want, atol=0.03, rtol=0.03)       # check_math.py:249-250
    np.testing.assert_allclose(total, want_total, atol=1e-5)
    # all selected: mean LSE is -inf everywhere and the merge is the identity
    full = ref.protected_selection(np.zeros((1, 4, 4, 4), np.float32), 0.0, 2, 4, 2)
    m_out, m_lse = ref.mean_tail(q, d, full, SCALE)
    assert (m_lse == -np.inf).all() and (m_out == 0).all()
    e_out, e_lse = ref.exact_attention(q, k, v, *ref.indices_from_mask(full), SCALE)
    o, l = ref.merge_exact_mean(e_out, e_lse, m_out, m_lse)
    np.testing.assert_array_equal(o, e_out)
    np.testing.assert_array_equal(l, e_lse)


def test_zero_dispersion_counterexample():
    """check_math.py:202-219: logits A = [2, -2], B = [5, 5]; value 1 on block A."""
    q = np.ones((1, 6, 1, 1), np.float32)
    k = np.array([2, -2, 5, 5, 0, 0], np.float32).reshape(1, 6, 1, 1)
    v = np.array([1, 1, 0, 0, 0, 0], np.float32).reshape(1, 6, 1, 1)
    d = ref.block_descriptors(k, v, block_size=2)
    idx = np.full((1, 3, 3, 1), 3, np.int64)
    cnt = np.zeros((1, 3, 1), np.int32)
    idx[0, 2, :2, 0] = [0, 1]
    cnt[0, 2, 0] = 2
    exact, _ = ref.exact_attention(q, k, v, idx, cnt, 1.0, block_size=2, precision="f64")
    none = np.zeros((1, 3, 3, 1), bool)
    mean, _ = ref.mean_tail(q, d, none, 1.0, block_size=2)
    e = (math.exp(2) + math.exp(-2)) / (math.exp(2) + math.exp(-2) + 2 * math.exp(5))
    assert float(exact[0, 4, 0, 0]) == pytest.approx(e, rel=4e-3)          # bf16-rounded output
    assert float(mean[0, 4, 0, 0]) == pytest.approx(2 / (2 + 2 * math.exp(5)), rel=1e-6)
    assert abs(e - float(mean[0, 4, 0, 0])) == pytest.approx(0.0180, abs=1e-4)


def test_merge_known_answers():
    eo = ref.bf16_round(rnd((1, 3, 2, 4), 31))
    mo = rnd((1, 3, 2, 4), 32)
    el = np.zeros((1, 3, 2), np.float32)
    o, l = ref.merge_exact_mean(eo, el, mo, np.full_like(el, -np.inf))
    np.testing.assert_array_equal(o, eo)
    np.testing.assert_array_equal(l, el)
    o, l = ref.merge_exact_mean(eo, el, mo, el)                 # equal LSEs: plain average
    np.testing.assert_array_equal(o, ref.bf16_round(((eo + mo) / 2).astype(np.float32)))
    np.testing.assert_allclose(l, math.log(2.0), rtol=1e-7)


# ------------------------------------------------------- accounting

def test_selection_accounting_brute_force():
    rng = np.random.default_rng(33)
    length, blocks = 300, 3
    sel = (rng.random((2, blocks, blocks, 3)) < 0.6) & np.tril(np.ones((blocks, blocks), bool))[None, :, :, None]
    acct = ref.selection_accounting(sel, length, 64, 32, "mean_native", 32)
    n = [128, 128, 44]
    pairs = tail = phys = 0
    for b, t, j, h in itertools.product(range(2), range(blocks), range(blocks), range(3)):
        if sel[b, t, j, h]:
            pairs += n[t] * n[j] if j < t else (n[t] * (n[t] + 1) // 2 if j == t else 0)
            phys += math.ceil(n[t] / 64) * math.ceil(128 / 32)
        elif j < t:
            tail += n[t]
    assert acct["exact_token_pairs"] == pairs
    assert acct["selected_block_entries"] == int(sel.sum())
    assert acct["mean_proxy_entries"] == tail
    assert acct["exact_physical_qk_tiles"] == phys
    assert acct["causal_token_pairs"] == 2 * 3 * length * (length + 1) // 2
    assert acct["selector_physical_qk_tiles"] == (1 + 1 + 1) * 2 * 3
    assert acct["mean_executed_logit_entries"] == 2 * length * 3 * blocks


# ------------------------------------------------------- whole layer

def test_attention_layer_method_relations():
    q, k, v = rnd((1, 300, 4, 16), 34), rnd((1, 300, 2, 16), 35), rnd((1, 300, 2, 16), 36)
    fp = ref.attention_layer(q, k, v, 0.25, "fp_v1", 0.5)
    mn = ref.attention_layer(q, k, v, 0.25, "mean_native", 0.5)
    np.testing.assert_array_equal(fp["selected"], mn["selected"])         # check_math.py:313-320
    dense = ref.attention_layer(q, k, v, 0.25, "dense")
    d_out, _ = dense_reference(q, k, v, 0.25)
    np.testing.assert_array_equal(dense["output"], ref.bf16_round(d_out.astype(np.float32)))
    for rescue in ("fp_v1_rescue", "fp_v1_rescue_v2"):                   # same V1 routing
        np.testing.assert_array_equal(ref.attention_layer(q, k, v, 0.25, rescue, 0.5)["selected"],
                                      fp["selected"])
    with pytest.raises(ValueError):
        ref.attention_layer(q, k, v, 0.25, "topk")


# ----------------------------------------------------------- rescue tail

def explicit_rescue_reference(q, k, v, selected, scale, remainder, block=128):
    """check_math.py:122-162: token-mask exact attention plus, per unselected
    full-history block, its argmax_j qbar.k_j token (and with ``remainder`` the
    mean K / V of the other B-1 tokens with multiplicity B-1), float64 loops."""
    _, sequence, heads, dim = q.shape
    group = heads // k.shape[2]
    keys = np.repeat(k[0], group, 1).astype(np.float64)
    values = np.repeat(v[0], group, 1).astype(np.float64)
    queries = q[0].astype(np.float64)
    pos = np.arange(sequence)
    out = np.zeros((sequence, heads, dim))
    lse = np.zeros((sequence, heads))
    for tile in range(selected.shape[1]):
        rows = np.arange(tile * block, min(sequence, (tile + 1) * block))
        for head in range(heads):
            allowed = selected[0, tile, pos // block, head][None, :] & (pos[None, :] <= rows[:, None])
            logits = [np.where(allowed, queries[rows, head] @ keys[:, head].T * scale, -np.inf)]
            parts = [values[:, head]]
            qbar = queries[rows, head].mean(axis=0)
            for key_block in range(tile):
                if selected[0, tile, key_block, head]:
                    continue
                span = slice(key_block * block, (key_block + 1) * block)
                bk, bv = keys[span, head], values[span, head]
                choice = int(np.argmax(bk @ qbar))
                logits.append(queries[rows, head] @ bk[choice][:, None] * scale)
                parts.append(bv[choice][None])
                if remainder:
                    rest = np.arange(block) != choice
                    logits.append(queries[rows, head] @ bk[rest].mean(axis=0)[:, None] * scale
                                  + np.log(block - 1.0))
                    parts.append(bv[rest].mean(axis=0)[None])
            z = np.concatenate(logits, axis=1)
            m = z.max(axis=1, keepdims=True)
            w = np.exp(z - m)
            lse[rows, head] = (m + np.log(w.sum(axis=1, keepdims=True)))[:, 0]
            out[rows, head] = (w / w.sum(axis=1, keepdims=True)) @ np.concatenate(parts, axis=0)
    return out[None], lse[None]


def _rescue_fixture():
    """check_math.py:252-262: 385 tokens (4 tiles, the last has one row), fixed mask."""
    q, k, v = rnd((1, 385, 4, 8), 40), rnd((1, 385, 2, 8), 41), rnd((1, 385, 2, 8), 42)
    sel = ref.protected_selection(np.zeros((1, 4, 4, 4), np.float32), 0.0, 2, 4, 2)
    sel[:, 2, 0, ::2] = False
    sel[:, 2, 1, 1::2] = False
    sel[:, 3, 1, :] = False
    return q, k, v, sel


@pytest.mark.parametrize("remainder", (False, True))
def test_exact_plus_rescue_against_check_math(remainder):
    q, k, v, sel = _rescue_fixture()
    idx, cnt = ref.indices_from_mask(sel)
    merged, total = ref.merge_exact_mean(*ref.exact_attention(q, k, v, idx, cnt, SCALE),
                                         *ref.rescue_tail(q, k, v, sel, SCALE, remainder=remainder))
    want, want_total = explicit_rescue_reference(q, k, v, sel, SCALE, remainder)
    np.testing.assert_allclose(merged, want, atol=0.03, rtol=0.03)       # check_math.py:281-282
    np.testing.assert_allclose(total, want_total, atol=1e-5)
    # rows of tiles 0-1 have no unselected history: the rescue LSE is -inf there
    _, r_lse = ref.rescue_tail(q, k, v, sel, SCALE, remainder=remainder)
    assert (r_lse[:, :256] == -np.inf).all() and np.isfinite(r_lse[:, 256:]).all()


def test_rescue_choice_loop_ties_and_future_invariance():
    q, k = rnd((1, 300, 4, 8), 43), rnd((1, 300, 2, 8), 44)
    choice = ref.rescue_choice(q, k)
    for t, j, h in itertools.product(range(3), range(3), range(4)):
        if j >= t:
            assert choice[0, t, j, h] == 0
            continue
        rows = q[0, t * 128:min(300, t * 128 + 128), h].astype(np.float64)
        qbar = rows.sum(axis=0) / len(rows)
        scores = k[0, j * 128:(j + 1) * 128, h // 2].astype(np.float64) @ qbar
        assert choice[0, t, j, h] == int(np.argmax(scores))
    # exact ties pick the first position: two identical maximal keys in block 0
    k2 = np.zeros((1, 300, 2, 8), np.float32)
    k2[0, 5, 0] = k2[0, 77, 0] = 1.0
    q2 = np.ones((1, 300, 4, 8), np.float32)
    assert ref.rescue_choice(q2, k2)[0, 1, 0, 0] == 5
    # all scores equal (zero keys): position 0
    assert ref.rescue_choice(q2, np.zeros_like(k2))[0, 2, 1, 3] == 0


@pytest.mark.parametrize("remainder", (False, True))
def test_rescue_future_kv_invariance_and_all_selected(remainder):
    q, k, v, sel = _rescue_fixture()
    out, lse = ref.rescue_tail(q, k, v, sel, SCALE, remainder=remainder)
    k2, v2 = k.copy(), v.copy()
    k2[:, 300:] *= 19                                                    # check_math.py:283-287
    v2[:, 300:] += 23
    out2, lse2 = ref.rescue_tail(q, k2, v2, sel, SCALE, remainder=remainder)
    np.testing.assert_array_equal(out2[:, :300], out[:, :300])
    np.testing.assert_array_equal(lse2[:, :300], lse[:, :300])
    full = ref.protected_selection(np.zeros((1, 4, 4, 4), np.float32), 0.0, 2, 4, 2)
    f_out, f_lse = ref.rescue_tail(q, k, v, full, SCALE, remainder=remainder)
    assert (f_lse == -np.inf).all() and (f_out == 0).all()
