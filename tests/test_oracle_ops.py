"""Pins the oracle's per-op math (CPU only).

Every check here is independent of the oracle's own formula: a known answer, a
closed form, an invariant, or a second implementation (torch's CPU kernels,
scipy). A plausible slip in the oracle -- a dropped term, a wrong sign or
index, a transposed operand, a missing rounding -- fails at least one of them.
"""
from __future__ import annotations

import math

import numpy as np
import pytest
import torch

from oracle import ops as O

RNG = np.random.default_rng(1234)


# --------------------------------------------------------------------------- bf16


def test_bf16_round_matches_torch_on_random_and_edge_values():
    vals = np.concatenate([
        RNG.standard_normal(20000).astype(np.float32) * 10.0,
        np.array([0.0, -0.0, 1.0, -1.0, 3.4e38, -3.4e38, 1e-40, -1e-40, np.inf, -np.inf],
                 dtype=np.float32),
        # exact ties: 1 + 2^-8 (half an ulp at 1) rounds to even (1.0); 1 + 3*2^-8 rounds up
        np.array([1 + 2 ** -8, 1 + 3 * 2 ** -8, -(1 + 2 ** -8)], dtype=np.float32),
    ])
    ours = O.bf16_round(vals)
    ref = torch.from_numpy(vals).to(torch.bfloat16).to(torch.float32).numpy()
    np.testing.assert_array_equal(ours, ref)
    assert O.bf16_round(np.array([1 + 2 ** -8], np.float32))[0] == 1.0
    assert O.bf16_round(np.array([1 + 3 * 2 ** -8], np.float32))[0] == 1 + 2 ** -6


def test_bf16_round_keeps_nan_and_bits_round_trip():
    assert np.isnan(O.bf16_round(np.array([np.nan], np.float32))[0])
    x = RNG.standard_normal(1000).astype(np.float32)
    np.testing.assert_array_equal(O.bf16_from_bits(O.bf16_bits(x)), O.bf16_round(x))
    assert O.bf16_bits(np.array([1.0], np.float32))[0] == 0x3F80
    assert O.bf16_bits(np.array([-2.0], np.float32))[0] == 0xC000


# --------------------------------------------------------------------------- RMSNorm


def test_rms_norm_constant_row_closed_form():
    c, eps = 3.0, 1e-6
    x = np.full((1, 64), c, np.float32)
    w = np.linspace(0.5, 1.5, 64).astype(np.float32)
    got = O.rms_norm(x, w, eps)
    want = c / math.sqrt(c * c + eps) * w.astype(np.float64)
    np.testing.assert_allclose(got[0], want, rtol=1e-6)


def test_rms_norm_matches_torch_and_fp64_truth():
    x = RNG.standard_normal((7, 1024)).astype(np.float32) * 4
    w = O.bf16_round(RNG.uniform(0.5, 1.5, 1024).astype(np.float32))
    got = O.rms_norm(x, w, 1e-6)
    ref = torch.nn.functional.rms_norm(torch.from_numpy(x), (1024,), torch.from_numpy(w),
                                       eps=1e-6).numpy()
    np.testing.assert_allclose(got, ref, rtol=2e-6, atol=2e-6)
    np.testing.assert_allclose(got, O.rms_norm64(x, w, 1e-6), rtol=2e-6, atol=2e-6)


def test_rms_norm_per_head_axis():
    """q/k norm runs over the last axis (head_dim) of [rows, heads, hd]."""
    q = RNG.standard_normal((3, 4, 128)).astype(np.float32)
    w = np.ones(128, np.float32)
    got = O.rms_norm(q, w, 1e-6)
    rms = np.sqrt(np.mean(got.astype(np.float64) ** 2, axis=-1))
    np.testing.assert_allclose(rms, 1.0, rtol=1e-5)


# --------------------------------------------------------------------------- RoPE


def test_rope_tables_known_values():
    cos, sin = O.rope_tables(np.array([0, 1, 7]), 128, 1e6)
    assert cos.shape == (3, 1, 128)
    np.testing.assert_array_equal(cos[0], 1.0)
    np.testing.assert_array_equal(sin[0], 0.0)
    # inv_freq[0] = 1: column 0 rotates by exactly the position
    np.testing.assert_allclose(cos[2, 0, 0], math.cos(7.0), rtol=1e-6)
    # last frequency 1/theta^(63/64), halves duplicated
    f63 = 1.0 / (1e6 ** (63 / 64))
    np.testing.assert_allclose(sin[1, 0, 63], math.sin(f63), rtol=1e-4)
    np.testing.assert_array_equal(cos[:, :, :64], cos[:, :, 64:])
    np.testing.assert_array_equal(sin[:, :, :64], sin[:, :, 64:])


def test_split_half_rope_is_complex_rotation():
    """out = x*cos + [-x2, x1]*sin rotates each pair (x_i, x_{i+64}) by pos*f_i."""
    pos = np.array([0, 5, 1000, 8191])
    x = RNG.standard_normal((4, 2, 128)).astype(np.float32)
    cos, sin = O.rope_tables(pos, 128, 1e6)
    got = O.apply_split_half_rope(x, cos, sin).astype(np.float64)
    inv = 1.0 / (1e6 ** (np.arange(64) / 64.0))
    z = x[..., :64].astype(np.float64) + 1j * x[..., 64:].astype(np.float64)
    rot = z * np.exp(1j * pos[:, None, None] * inv[None, None, :])
    np.testing.assert_allclose(got[..., :64], rot.real, atol=2e-3)
    np.testing.assert_allclose(got[..., 64:], rot.imag, atol=2e-3)


def test_rope_relative_position_invariance():
    """<rope(q, m), rope(k, n)> depends only on m - n."""
    q = RNG.standard_normal((1, 1, 128)).astype(np.float32)
    k = RNG.standard_normal((1, 1, 128)).astype(np.float32)

    def dot(m, n):
        cm, sm = O.rope_tables(np.array([m]), 128, 1e6)
        cn, sn = O.rope_tables(np.array([n]), 128, 1e6)
        a = O.apply_split_half_rope(q, cm, sm).astype(np.float64)
        b = O.apply_split_half_rope(k, cn, sn).astype(np.float64)
        return float((a * b).sum())

    np.testing.assert_allclose(dot(10, 3), dot(107, 100), rtol=1e-4)


# --------------------------------------------------------------------------- SwiGLU


def test_swiglu_matches_torch_silu():
    g = RNG.standard_normal(4096).astype(np.float32) * 6
    u = RNG.standard_normal(4096).astype(np.float32)
    ref = (torch.nn.functional.silu(torch.from_numpy(g)) * torch.from_numpy(u)).numpy()
    np.testing.assert_allclose(O.swiglu(g, u), ref, rtol=1e-5, atol=1e-6)
    assert O.swiglu(np.float32([0.0]), np.float32([5.0]))[0] == 0.0


# --------------------------------------------------------------------------- q4


def test_q4_unpack_known_answer_words():
    """MLX packing: low nibble first along K (word j holds k = 8j..8j+7)."""
    w = np.array([[0x76543210, 0xFEDCBA98]], dtype=np.uint32)
    np.testing.assert_array_equal(O.q4_unpack(w)[0], np.arange(16))
    w2 = np.array([[0x0000000F, 0xF0000000]], dtype=np.uint32)
    want = np.zeros(16, np.uint8)
    want[0], want[15] = 15, 15
    np.testing.assert_array_equal(O.q4_unpack(w2)[0], want)


def test_q4_pack_round_trip():
    nib = RNG.integers(0, 16, size=(5, 128), dtype=np.uint8)
    np.testing.assert_array_equal(O.q4_unpack(O.q4_pack(nib)), nib)
    assert O.q4_pack(np.arange(8, dtype=np.uint8)[None])[0, 0] == 0x76543210


def test_q4_dequant_group_boundaries():
    """scale/bias index is k // 64: columns 63 and 64 use different groups."""
    nib = np.full((2, 128), 3, np.uint8)
    nib[1, 64] = 15
    scales = np.array([[0.5, 2.0], [0.25, 4.0]], np.float32)
    biases = np.array([[-1.0, 10.0], [0.0, -8.0]], np.float32)
    w = O.q4_dequant(O.q4_pack(nib), scales, biases)
    assert w[0, 63] == 0.5 * 3 - 1.0 and w[0, 64] == 2.0 * 3 + 10.0
    assert w[1, 0] == 0.25 * 3 and w[1, 64] == 4.0 * 15 - 8.0


def test_q4_linear_matches_brute_force_loop():
    n, k, m = 3, 128, 2
    nib = RNG.integers(0, 16, size=(n, k), dtype=np.uint8)
    words = O.q4_pack(nib)
    scales = O.bf16_round(RNG.uniform(0.005, 0.02, (n, k // 64)).astype(np.float32))
    biases = O.bf16_round(RNG.uniform(-0.1, 0.1, (n, k // 64)).astype(np.float32))
    x = RNG.standard_normal((m, k)).astype(np.float32)
    y = O.linear(x, O.Q4Weight(words, scales, biases), None, weight_kind="q4")
    for i in range(m):
        for j in range(n):
            acc = 0.0
            for kk in range(k):
                word = int(words[j, kk // 8])
                q = (word >> (4 * (kk % 8))) & 0xF
                acc += float(x[i, kk]) * (float(scales[j, kk // 64]) * q +
                                          float(biases[j, kk // 64]))
            assert abs(y[i, j] - acc) <= 1e-5 * max(1.0, abs(acc))


# --------------------------------------------------------------------------- linear


def test_round_half_away_known_values():
    x = np.array([2.5, -2.5, 0.5, -0.5, 1.5, 0.49999997, -0.49999997, 3.4999998, 7.0, -0.0],
                 dtype=np.float32)
    want = np.array([3, -3, 1, -1, 2, 0, 0, 3, 7, 0], dtype=np.float32)
    assert np.array_equal(O.round_half_away(x), want)
    # off the .5 points it is numpy's nearest rounding
    r = np.random.default_rng(0).normal(0, 20, 10000).astype(np.float32)
    r = r[np.abs(r - np.trunc(r)) != 0.5]
    assert np.array_equal(O.round_half_away(r), np.round(r))


def test_q4_quantize_exact_affine_ramps():
    q = np.random.default_rng(1).integers(0, 16, (3, 128))
    q[:, 0], q[:, 64], q[:, 1], q[:, 65] = 0, 0, 15, 15  # both extremes in every group
    # |w_min| > |w_max|: positive scale, bias = w_min
    w = (-1.0 + 0.125 * q).astype(np.float32)
    wq, s, b = O.q4_quantize(w)
    assert np.array_equal(O.q4_unpack(wq), q)
    assert np.all(s == 0.125) and np.all(b == -1.0)
    assert np.array_equal(O.q4_dequant(wq, s, b), w)
    # |w_max| >= |w_min|: the scale is negated and the bias is w_max
    w2 = (1.0 - 0.125 * q).astype(np.float32)
    wq2, s2, b2 = O.q4_quantize(w2)
    assert np.array_equal(O.q4_unpack(wq2), q)
    assert np.all(s2 == -0.125) and np.all(b2 == 1.0)
    assert np.array_equal(O.q4_dequant(wq2, s2, b2), w2)


def test_q4_quantize_constant_and_zero_groups():
    w = np.zeros((2, 128), dtype=np.float32)
    w[1, :64] = 0.3
    w[1, 64:] = -2.0
    wq, s, b = O.q4_quantize(w)
    assert np.all(O.q4_unpack(wq) == 0)
    # an all-zero group keeps the negated minimum scale and a zero bias
    assert s[0, 0] == O.bf16_round(np.float32(-1e-7)) and b[0, 0] == 0.0
    # a constant group is its bias exactly (bf16 of the constant)
    assert b[1, 0] == O.bf16_round(np.float32(0.3)) and b[1, 1] == -2.0
    deq = O.q4_dequant(wq, s, b)
    assert np.array_equal(deq[1], O.bf16_round(w[1]))


def test_q4_quantize_rounds_halves_away_from_zero():
    # scale 0.125, bias -1: -0.6875 sits at q = 2.5 exactly and goes to 3
    w = np.full((1, 64), 0.0, dtype=np.float32)
    w[0, 0], w[0, 1], w[0, 2] = -1.0, 0.875, -0.6875
    w[0, 3:] = -1.0 + 0.125 * (np.arange(61) % 16)
    q = O.q4_unpack(O.q4_quantize(w)[0])[0]
    assert q[2] == 3


def test_q4_quantize_is_nearest_grid_point():
    rng = np.random.default_rng(2)
    w = (rng.normal(0, 0.02, (16, 256)) + rng.normal(0, 0.01, (16, 1))).astype(np.float32)
    w[3, :64] = np.abs(w[3, :64])   # one-signed groups
    w[4, 64:128] = -np.abs(w[4, 64:128])
    wq, s, b, s32, b32 = O.q4_quantize(w, return_fp32=True)
    wb = O.bf16_round(w).astype(np.float64).reshape(16, 4, 64)
    q = O.q4_unpack(wq).astype(np.float64).reshape(16, 4, 64)
    grid = b32[..., None, None] + s32[..., None, None] * np.arange(16.0)  # [16, 4, 1, 16]
    dist = np.abs(wb[..., None] - grid)                                     # [16, 4, 64, 16]
    best = dist.min(axis=-1)
    chosen = np.take_along_axis(dist, q[..., None].astype(np.int64), axis=-1)[..., 0]
    # brute force over the 16 levels: the chosen level is a nearest one (fp32 slack)
    assert np.all(chosen <= best + 1e-6 * np.abs(s32)[..., None])
    # unclamped levels are within half a step, clamped ones within a step
    err = np.abs(wb - (b32[..., None] + s32[..., None] * q))
    assert np.all(err <= np.abs(s32)[..., None] * np.where(q == 15, 1.0, 0.5) * (1 + 1e-5))
    # the edge value sits exactly on the fp32 grid (bias = edge)
    edge_side = np.abs(wb.min(-1)) > np.abs(wb.max(-1))
    edge = np.where(edge_side, wb.min(-1), wb.max(-1))
    assert np.all(b32 == edge)
    # zero lies on the grid: bias / scale is (minus) an integer level (the q0
    # adjustment), not the raw (w_max - w_min) / 15 step
    ratio = b32.astype(np.float64) / s32
    assert np.all(np.abs(ratio - np.round(ratio)) < 1e-4)
    raw = (wb.max(-1) - wb.min(-1)) / 15
    assert np.mean(np.abs(np.abs(s32) - raw) > 1e-6 * raw) > 0.5
    # stored scale/bias are the bf16 roundings of the fp32 ones
    assert np.array_equal(s, O.bf16_round(s32)) and np.array_equal(b, O.bf16_round(b32))


def test_q4_quantize_input_is_rounded_to_bf16_first():
    w = np.random.default_rng(3).normal(0, 0.02, (4, 64)).astype(np.float32)
    for a, b in zip(O.q4_quantize(w), O.q4_quantize(O.bf16_round(w))):
        assert np.array_equal(a, b)


def test_bf16_linear_matches_torch_bf16_matmul():
    """(x.astype(bf16) @ W.T) with a bf16 result, as torch's bf16 CPU matmul."""
    x = RNG.standard_normal((5, 96)).astype(np.float32)
    w = O.bf16_round(RNG.standard_normal((7, 96)).astype(np.float32) * 0.05)
    got = O.linear(x, w, None, weight_kind="bf16")
    ref = (torch.from_numpy(x).bfloat16() @ torch.from_numpy(w).bfloat16().T).float().numpy()
    # accumulation order may differ by one bf16 rounding step
    ulp = 2.0 ** (np.floor(np.log2(np.maximum(np.abs(ref), 1e-30))) - 7)
    assert np.all(np.abs(got - ref) <= ulp + 1e-30)


def test_bf16_linear_rounds_input_and_output():
    """K=1 exact products: the activation and the product are both rounded."""
    x = np.array([[1.0 + 2 ** -9]], np.float32)     # rounds to 1.0 in bf16
    w = np.array([[1.0 + 2 ** -7]], np.float32)     # a bf16 value
    assert O.linear(x, w, None, weight_kind="bf16")[0, 0] == np.float32(1.0 + 2 ** -7)
    x2 = np.array([[1.0 + 2 ** -7]], np.float32)
    # (1+2^-7)^2 = 1 + 2^-6 + 2^-14 -> bf16 1 + 2^-6
    assert O.linear(x2, w, None, weight_kind="bf16")[0, 0] == np.float32(1.0 + 2 ** -6)
    b = np.array([0.5], np.float32)
    assert O.linear(x2, w, b, weight_kind="bf16")[0, 0] == np.float32(1.5 + 2 ** -6)


def test_fp32_linear_bias_and_orientation():
    x = np.array([[1.0, 2.0, 3.0]], np.float32)
    w = np.array([[1.0, 0.0, 0.0], [0.0, 0.0, 1.0]], np.float32)   # [N=2, K=3]
    np.testing.assert_array_equal(O.linear(x, w, np.float32([10, 20]), weight_kind="fp32"),
                                  [[11.0, 23.0]])


# --------------------------------------------------------------------------- masks


def test_d2f_visible_staircase_and_prompt():
    vis = O.d2f_visible(np.arange(70), 70, prompt_len=0, block_size=32)
    ii, jj = np.meshgrid(np.arange(70), np.arange(70), indexing="ij")
    np.testing.assert_array_equal(vis, (jj // 32) <= (ii // 32))
    # prompt columns are visible to every row; a prompt row sees only the prompt
    vis = O.d2f_visible(np.arange(10), 10, prompt_len=4, block_size=3)
    assert vis[:, :4].all()
    assert not vis[0, 4:].any()
    assert vis[4, 4:7].all() and not vis[4, 7:].any()   # first block: bidirectional inside
    assert vis[9].all()


# --------------------------------------------------------------------------- attention


def _torch_sdpa(q, k, v, visible):
    group = q.shape[1] // k.shape[1]
    qt = torch.from_numpy(q).double().transpose(0, 1)
    kt = torch.from_numpy(k).double().repeat_interleave(group, dim=1).transpose(0, 1)
    vt = torch.from_numpy(v).double().repeat_interleave(group, dim=1).transpose(0, 1)
    mask = None if visible is None else torch.from_numpy(visible)
    o = torch.nn.functional.scaled_dot_product_attention(qt, kt, vt, attn_mask=mask)
    return o.transpose(0, 1).reshape(q.shape[0], -1).numpy()


@pytest.mark.parametrize("masked", [False, True])
def test_attention_matches_torch_sdpa_gqa(masked):
    q = RNG.standard_normal((40, 4, 128)).astype(np.float32)
    k = RNG.standard_normal((40, 2, 128)).astype(np.float32)
    v = RNG.standard_normal((40, 2, 128)).astype(np.float32)
    vis = O.d2f_visible(np.arange(40), 40, prompt_len=8, block_size=16) if masked else None
    np.testing.assert_allclose(O.attention(q, k, v, visible=vis), _torch_sdpa(q, k, v, vis),
                               rtol=1e-10, atol=1e-10)


def test_attention_key_permutation_invariance_and_limits():
    q = RNG.standard_normal((3, 2, 128))
    k = RNG.standard_normal((9, 1, 128))
    v = RNG.standard_normal((9, 1, 128))
    perm = RNG.permutation(9)
    np.testing.assert_allclose(O.attention(q, k, v), O.attention(q, k[perm], v[perm]),
                               rtol=1e-12, atol=1e-12)
    # one key: output is that key's value for every query head
    o = O.attention(q, k[:1], v[:1]).reshape(3, 2, 128)
    np.testing.assert_allclose(o, np.broadcast_to(v[0, 0], (3, 2, 128)), rtol=1e-12)
    # identical keys: uniform weights -> mean of the values
    kk = np.broadcast_to(k[:1], k.shape).copy()
    o = O.attention(q, kk, v).reshape(3, 2, 128)
    np.testing.assert_allclose(o[0, 0], v[:, 0].mean(axis=0), rtol=1e-10)


# --------------------------------------------------------------------------- scoring


def test_required_raw_row():
    assert [O.required_raw_row(p, logits_convention="dream_ar_shift") for p in (0, 1, 9)] == \
        [0, 0, 8]
    assert O.required_raw_row(9, logits_convention="raw") == 9
    with pytest.raises(ValueError):
        O.required_raw_row(1, logits_convention="shifted")


def test_raw_max_prob_closed_forms():
    logits = np.array([[0.0, math.log(3.0)],       # p = 3/4 at index 1
                       [2.0, 2.0],                 # tie: p = 1/2, first index
                       [-1e30, 0.0]], np.float32)  # underflow: p = 1
    scores, tokens = O.raw_max_prob(logits)
    np.testing.assert_allclose(scores, [0.75, 0.5, 1.0], rtol=1e-7)
    assert tokens == [1, 0, 1]
    big = RNG.standard_normal((4, 151936)).astype(np.float32) * 3
    s, t = O.raw_max_prob(big)
    from scipy.special import softmax
    ref = softmax(big.astype(np.float64), axis=-1)
    np.testing.assert_allclose(s, ref.max(axis=-1), rtol=1e-12)
    assert t == ref.argmax(axis=-1).tolist()
    # shift invariance of the float64 softmax
    s2, t2 = O.raw_max_prob(big.astype(np.float64) + 100.0)
    np.testing.assert_allclose(s2, s, rtol=1e-12)
    assert t2 == t


def test_topk_count_choices_order():
    conf = np.array([0.1, 0.9, 0.5, 0.7, 0.3])
    assert O.topk_count_choices(conf, 3) == [1, 3, 2]
    assert O.topk_count_choices(conf, 0) == []
    assert O.topk_count_choices(conf, 9) == [1, 3, 2, 4, 0]


# --------------------------------------------------------------------------- sampling


def test_mix64_matches_published_splitmix64_sequence():
    """splitmix64 from state 0: outputs are mix64(i * 0x9E3779B97F4A7C15), i = 1.."""
    want = [0xE220A8397B1DCDAF, 0x6E789E6AA1B965F4, 0x06C45D188009454F, 0xF88BB8A8724C81EC]
    got = [O.mix64(i * O.SAMPLING_STEP) for i in range(1, 5)]
    assert got == want


def test_sampling_noise_is_gumbel():
    """23-bit uniforms mapped through -log(-log u): Gumbel(0,1) mean ~ 0.5772, var pi^2/6."""
    g = O.sampling_noise(7, 0, 3, 20000).astype(np.float64)
    assert abs(g.mean() - 0.5772) < 0.03
    assert abs(g.var() - math.pi ** 2 / 6) < 0.08
    # keyed: another step or position gives different noise, the same key the same
    assert not np.array_equal(g[:64], O.sampling_noise(7, 1, 3, 64))
    assert not np.array_equal(g[:64], O.sampling_noise(7, 0, 4, 64))
    np.testing.assert_array_equal(g[:64], O.sampling_noise(7, 0, 3, 64))


def test_sampled_max_prob_reduces_to_greedy_at_zero_temperature():
    logits = RNG.standard_normal((3, 300)).astype(np.float32)
    s, t = O.sampled_max_prob(logits, temperature=0.0, seed=1, step=0, positions=[4, 5, 6])
    s0, t0 = O.raw_max_prob(logits)
    assert t == t0
    np.testing.assert_allclose(s, s0, rtol=1e-12)
