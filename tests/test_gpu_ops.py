"""GPU parity of the per-op kernels against the oracle (configs 2 and 3 shapes).

Each test prints the case it runs before touching the GPU.
"""
from __future__ import annotations

import math

import numpy as np
import pytest

from oracle import ops as O

torch = pytest.importorskip("torch")

pytestmark = pytest.mark.gpu


def _say(*a):
    print("[case]", *a, flush=True)


def _q4_case(n, k, seed, centred=False):
    from diffusorrt_amd import synthetic as syn

    gen = torch.Generator().manual_seed(seed)
    q = syn.random_q4(gen, n, k, scale_lo=0.005, scale_hi=0.02, centred=centred)
    return gen, q


# ---------------------------------------------------------------- q4 linear (config 3)

Q4_SHAPES = [(1024, 1024), (3072, 1024), (1024, 3072), (18944, 3584), (3584, 18944)]


@pytest.mark.parametrize("m", [32, 128])
@pytest.mark.parametrize("n,k", Q4_SHAPES)
def test_q4_linear_config3(m, n, k):
    from diffusorrt_amd import kernels

    _say("q4_linear", m, n, k)
    gen, q = _q4_case(n, k, seed=2)
    x = torch.randn((m, k), generator=gen).to(torch.bfloat16)
    w = kernels.DeviceQ4Weight(q.w_q.cuda(), q.scales.cuda(), q.biases.cuda())
    y = kernels.linear(x.cuda(), w).cpu().numpy().astype(np.float64)
    W = O.Q4Weight(q.w_q.numpy().view(np.uint32), q.scales.float().numpy(),
                   q.biases.float().numpy())
    xf = x.float().numpy()
    x16 = xf.astype(np.float16).astype(np.float64)
    if m <= 32:
        # what the weight-streaming kernels multiply: the activation as fp16 hi +
        # lo (a bf16 input is exact in the hi part), exact integer nibbles (scale
        # and bias applied in fp32)
        ref16 = O.q4_linear64(x16, W)
    else:
        # the large-M kernels dequantize each weight once to fp16: s * q + b with
        # a single rounding (exact products and sum in float64, then fp16)
        w16 = O.q4_dequant(W.w_q, W.scales, W.biases, dtype=np.float64).astype(np.float16)
        ref16 = x16 @ w16.astype(np.float64).T
    scale = np.abs(ref16).max()
    err16 = np.abs(y - ref16).max() / scale
    # the reference's semantics: fp32 activation into mx.quantized_matmul
    ref = O.q4_linear64(xf, W)
    err = np.abs(y - ref).max() / np.abs(ref).max()
    _say(f"  err_vs_fp16_input={err16:.2e} err_vs_reference={err:.2e}")
    assert err16 < 2e-5  # fp32 accumulation only
    # bf16 inputs are exact in fp16: accumulation (and for m > 32 the fp16 weights)
    assert err < 2e-3


@pytest.mark.parametrize("k", [192, 1024])
def test_q4_linear_large_m_ragged_with_bias(k):
    """The large-M kernels on ragged shapes: 200 rows (a partial 128-row tile),
    352 columns (a partial 256-column tile, 11 n-tiles), with a bias, against
    fp16-dequantized weights in float64. k = 192 (3 groups) runs one K slice with
    the bias in the kernel; k = 1024 splits K and adds the bias in the slice sum."""
    from diffusorrt_amd import kernels

    m, n = 200, 352
    _say("q4_linear large-M ragged", m, n, k)
    # independent biases (centred ones, b = -8s, make s * q + b exact in fp16)
    gen, q = _q4_case(n, k, seed=8, centred=False)
    x = torch.randn((m, k), generator=gen)
    bias = (torch.randn(n, generator=gen) * 0.1).to(torch.bfloat16)
    w = kernels.DeviceQ4Weight(q.w_q.cuda(), q.scales.cuda(), q.biases.cuda())
    y = kernels.linear(x.cuda(), w, bias.cuda()).cpu().numpy().astype(np.float64)
    W = O.Q4Weight(q.w_q.numpy().view(np.uint32), q.scales.float().numpy(),
                   q.biases.float().numpy())
    w16 = O.q4_dequant(W.w_q, W.scales, W.biases, dtype=np.float64).astype(np.float16)
    # the fp32 activation enters as fp16 hi + lo: ~22 significant bits
    x64 = x.numpy().astype(np.float64)
    ref = x64 @ w16.astype(np.float64).T + bias.float().numpy()
    assert np.abs(y - ref).max() / np.abs(ref).max() < 2e-5
    # the bound separates fp16-rounded weights from exact ones, and an fp16
    # activation from the hi + lo pair: a kernel that skipped or misplaced either
    # would not pass it
    exact = O.q4_linear64(x64, W) + bias.float().numpy()
    assert np.abs(exact - ref).max() / np.abs(ref).max() > 2e-5
    x16 = x.numpy().astype(np.float16).astype(np.float64)
    act16 = x16 @ w16.astype(np.float64).T + bias.float().numpy()
    assert np.abs(act16 - ref).max() / np.abs(ref).max() > 2e-5


@pytest.mark.parametrize("m,n,k", [(1, 18944, 3584), (9, 18944, 3584), (17, 3584, 18944)])
def test_q4_linear_stream_ragged_rows_fp32_with_bias(m, n, k):
    """The weight-streaming kernels (<= 32 rows, >= 8M weights) on ragged row
    counts with an fp32 input (a nonzero lo plane) and a bias: 1 and 9 rows over
    a 3-slice plan with 16-group chunks, 17 rows over 8 slices of 37 groups
    (8-group chunks), against the exact q4 linear in float64."""
    from diffusorrt_amd import kernels

    _say("q4_linear stream ragged fp32 + bias", m, n, k)
    gen, q = _q4_case(n, k, seed=11, centred=False)
    x = torch.randn((m, k), generator=gen)
    bias = (torch.randn(n, generator=gen) * 0.1).to(torch.bfloat16)
    w = kernels.DeviceQ4Weight(q.w_q.cuda(), q.scales.cuda(), q.biases.cuda())
    y = kernels.linear(x.cuda(), w, bias.cuda()).cpu().numpy().astype(np.float64)
    W = O.Q4Weight(q.w_q.numpy().view(np.uint32), q.scales.float().numpy(),
                   q.biases.float().numpy())
    x64 = x.numpy().astype(np.float64)
    ref = O.q4_linear64(x64, W) + bias.float().numpy()
    err = np.abs(y - ref).max() / np.abs(ref).max()
    # an fp16-only activation (no lo plane) misses the bound by a wide margin
    x16 = x.numpy().astype(np.float16).astype(np.float64)
    err16 = np.abs(O.q4_linear64(x16, W) + bias.float().numpy() - ref).max() / np.abs(ref).max()
    _say(f"  err={err:.2e} (fp16-only activation would be {err16:.2e})")
    assert err < 2e-5
    assert err16 > 2e-5


def test_q4_linear_fp32_input_and_bias():
    from diffusorrt_amd import kernels

    m, n, k = 5, 96, 192  # ragged rows, 3 n-tiles, 3 groups
    _say("q4_linear fp32 ragged", m, n, k)
    gen, q = _q4_case(n, k, seed=7, centred=True)
    x = torch.randn((m, k), generator=gen)
    bias = (torch.randn(n, generator=gen) * 0.1).to(torch.bfloat16)
    w = kernels.DeviceQ4Weight(q.w_q.cuda(), q.scales.cuda(), q.biases.cuda())
    y = kernels.linear(x.cuda(), w, bias.cuda()).cpu().numpy().astype(np.float64)
    W = O.Q4Weight(q.w_q.numpy().view(np.uint32), q.scales.float().numpy(),
                   q.biases.float().numpy())
    # fp32 activation as fp16 hi + lo, exact nibbles: the reference's fp32 linear
    ref = O.q4_linear64(x.numpy().astype(np.float64), W) + bias.float().numpy()
    err = np.abs(y - ref).max() / np.abs(ref).max()
    _say(f"  err_vs_fp32_input={err:.2e}")
    assert err < 2e-5


@pytest.mark.parametrize("m,n,k", [(32, 1024, 1024), (128, 3072, 1024), (3, 64, 2048)])
def test_bf16_linear(m, n, k):
    from diffusorrt_amd import kernels

    _say("bf16_linear", m, n, k)
    gen = torch.Generator().manual_seed(11)
    wt = (torch.randn((n, k), generator=gen) * 0.02).to(torch.bfloat16)
    x = torch.randn((m, k), generator=gen)
    y = kernels.linear(x.cuda(), kernels.DeviceBF16Weight(wt.cuda())).cpu().numpy()
    ref = O.linear(x.numpy(), wt.float().numpy(), None, weight_kind="bf16")
    # both round the same fp32 sum to bf16: equal except at rounding boundaries
    exact = np.mean(y == ref)
    rel = np.abs(y.astype(np.float64) - ref).max() / np.abs(ref).max()
    _say(f"  exact_frac={exact:.4f} rel={rel:.2e}")
    assert exact > 0.97
    assert rel < 1e-2


# ---------------------------------------------------------------- attention (config 2)

def _attention_inputs(L, seed=1, rows=32, hq=16, hkv=8):
    gen = torch.Generator().manual_seed(seed)
    q = torch.randn((rows, hq, 128), generator=gen).to(torch.bfloat16)
    k = torch.randn((L + rows, hkv, 128), generator=gen).to(torch.bfloat16)
    v = torch.randn((L + rows, hkv, 128), generator=gen).to(torch.bfloat16)
    return q, k, v


@pytest.mark.parametrize("L", [512, 2048, 8192])
def test_block_attention_config2_bf16(L):
    from diffusorrt_amd.kernels import PrefixKVCache

    _say("attention bf16 config2 L=", L)
    q, k, v = _attention_inputs(L)
    cache = PrefixKVCache(1, 8, L + 32, dtype="bf16")
    cache.store(0, k.cuda(), v.cuda(), 0)
    out = cache.attention(0, q.cuda(), n_keys=L + 32, row_pos0=L, kind="bidirectional",
                          out_dtype=torch.bfloat16)
    got = out.float().cpu().numpy().astype(np.float64)
    ref = O.attention(q.float().numpy(), k.float().numpy(), v.float().numpy())
    err = np.abs(got - ref).max() / np.abs(ref).max()
    mean_rel = np.mean(np.abs(got - ref)) / np.mean(np.abs(ref))
    _say(f"  max_err={err:.2e} mean_rel={mean_rel:.2e}")
    assert err < 2e-2
    assert mean_rel < 6e-3


@pytest.mark.parametrize("dtype,L,rows", [("f16", 8192, 64), ("bf16", 2048, 64), ("f16", 160, 64),
                                          ("bf16", 100, 32), ("f16", 0, 32)])
def test_block_attention_decode_shapes(dtype, L, rows):
    """64 rows over a prefix (a block's first step carrying the commit of the
    block before it): 128 query vectors per KV head, four query tiles, eight
    consumer waves; and up to 256 keys (one key range, whose work-groups write
    the output without the range combine), against the oracle on the cache's
    rounding."""
    from diffusorrt_amd.kernels import PrefixKVCache

    _say("attention rows", rows, dtype, "L=", L)
    q, k, v = _attention_inputs(L, seed=7, rows=rows)
    cache = PrefixKVCache(1, 8, L + rows, dtype=dtype)
    tdt = torch.float16 if dtype == "f16" else torch.bfloat16
    cache.store(0, k.float().cuda(), v.float().cuda(), 0)  # bf16 values: exact in either cache
    odt = torch.float32 if dtype == "f16" else torch.bfloat16
    out = cache.attention(0, q.to(tdt).cuda(), n_keys=L + rows, row_pos0=L, kind="bidirectional",
                          out_dtype=odt)
    got = out.float().cpu().numpy().astype(np.float64)
    ref = O.attention(q.to(tdt).double().numpy(), k.to(tdt).double().numpy(),
                      v.to(tdt).double().numpy())
    err = np.abs(got - ref).max() / np.abs(ref).max()
    _say(f"  max_err={err:.2e}")
    # bf16 outputs add their own rounding: half an ulp, up to 2^-8 of a value
    assert err < 3e-3 + (2.0 ** -8 if odt == torch.bfloat16 else 0.0)


@pytest.mark.parametrize("hq,hkv", [(4, 2), (8, 4)])
def test_block_attention_many_key_ranges(hq, hkv):
    """Few KV heads over an 8K prefix: the decode attention splits each head's keys
    into 64-65 ranges (more than 32, the combine's second statistics form, and
    range batches past the first with a ragged last one)."""
    from diffusorrt_amd.kernels import PrefixKVCache

    L = 8192
    _say("attention bf16 many ranges hq/hkv=", hq, hkv)
    q, k, v = _attention_inputs(L, seed=3, hq=hq, hkv=hkv)
    cache = PrefixKVCache(1, hkv, L + 32, dtype="bf16")
    cache.store(0, k.cuda(), v.cuda(), 0)
    out = cache.attention(0, q.cuda(), n_keys=L + 32, row_pos0=L, kind="bidirectional",
                          out_dtype=torch.bfloat16)
    got = out.float().cpu().numpy().astype(np.float64)
    ref = O.attention(q.float().numpy(), k.float().numpy(), v.float().numpy())
    err = np.abs(got - ref).max() / np.abs(ref).max()
    mean_rel = np.mean(np.abs(got - ref)) / np.mean(np.abs(ref))
    _say(f"  max_err={err:.2e} mean_rel={mean_rel:.2e}")
    assert err < 2e-2
    assert mean_rel < 6e-3


@pytest.mark.parametrize("kind,rows,pos0,L", [("d2f_hybrid", 96, 64, 160),
                                              ("d2f_hybrid", 32, 8192, 8224),
                                              ("bidirectional", 100, 0, 100)])
def test_attention_masks_f16(kind, rows, pos0, L):
    from diffusorrt_amd.kernels import PrefixKVCache

    _say("attention f16", kind, rows, pos0, L)
    gen = torch.Generator().manual_seed(5)
    q = torch.randn((rows, 16, 128), generator=gen)
    k = torch.randn((L, 8, 128), generator=gen)
    v = torch.randn((L, 8, 128), generator=gen)
    cache = PrefixKVCache(1, 8, L, dtype="f16")
    cache.store(0, k.cuda(), v.cuda(), 0)
    geom = (0, 32) if kind == "d2f_hybrid" else None
    out = cache.attention(0, q.to(torch.float16).cuda(), n_keys=pos0 + rows, row_pos0=pos0,
                          kind=kind, mask_geometry=geom)
    got = out.cpu().numpy().astype(np.float64)
    q16 = q.numpy().astype(np.float16).astype(np.float64)
    k16 = k.numpy().astype(np.float16).astype(np.float64)
    v16 = v.numpy().astype(np.float16).astype(np.float64)
    vis = None
    if kind == "d2f_hybrid":
        vis = O.d2f_visible(np.arange(pos0, pos0 + rows), pos0 + rows, prompt_len=0, block_size=32)
    ref = O.attention(q16, k16[:pos0 + rows], v16[:pos0 + rows], visible=vis)
    err = np.abs(got - ref).max() / np.abs(ref).max()
    _say(f"  max_err={err:.2e}")
    assert err < 3e-3


# ---------------------------------------------------------------- small ops

def test_rms_norm_rope_swiglu():
    from diffusorrt_amd import kernels

    _say("rms_norm/rope/swiglu")
    gen = torch.Generator().manual_seed(3)
    x = torch.randn((37, 1024), generator=gen) * 3
    w = (1 + 0.1 * torch.randn(1024, generator=gen)).to(torch.bfloat16)
    y = kernels.rms_norm(x.cuda(), w.cuda(), 1e-6).cpu().numpy()
    ref = O.rms_norm64(x.numpy(), w.float().numpy(), 1e-6)
    assert np.abs(y - ref).max() < 1e-5 * np.abs(ref).max() * 10

    xr = torch.randn((9, 4, 128), generator=gen)
    pos = np.arange(100, 109)
    cos, sin = O.rope_tables(pos, 128, 1e6)
    yr = kernels.rope(xr.cuda(), torch.from_numpy(cos), torch.from_numpy(sin)).cpu().numpy()
    refr = O.apply_split_half_rope(xr.numpy(), cos, sin)
    assert np.abs(yr - refr).max() < 1e-5

    g = torch.randn(5000, generator=gen) * 4
    u = torch.randn(5000, generator=gen)
    ys = kernels.swiglu(g.cuda(), u.cuda()).cpu().numpy()
    refs = O.swiglu(g.numpy(), u.numpy())
    assert np.abs(ys - refs).max() < 1e-5 * max(1.0, np.abs(refs).max())


# ---------------------------------------------------------------- LM head + scoring

@pytest.mark.parametrize("kind,rows,n", [("q4", 32, 151936), ("q4", 20, 8256), ("q4", 45, 8256),
                                          ("bf16", 32, 151936)])
def test_lm_head_scores_tokens(kind, rows, n):
    """The full 151936-column head and a 129-block one (ragged column ranges per
    work-group), one 32-row tile, a partial tile and two tiles."""
    from diffusorrt_amd import _lib, kernels
    from diffusorrt_amd import synthetic as syn
    import ctypes as C

    k = 1024
    _say("lm_head", kind, rows, n, k)
    gen = torch.Generator().manual_seed(9)
    x = torch.randn((rows, k), generator=gen)
    lib = _lib.load()
    scores = torch.empty(rows, dtype=torch.float64, device="cuda")
    tokens = torch.empty(rows, dtype=torch.int32, device="cuda")
    logits = torch.empty((rows, n), dtype=torch.float32, device="cuda")
    ws_b = lib.drt_op_lm_head_workspace_bytes(rows, n, k)
    ws = torch.empty(ws_b, dtype=torch.uint8, device="cuda")
    xc = x.cuda()
    if kind == "q4":
        q = syn.random_q4(gen, n, k)
        w = kernels.DeviceQ4Weight(q.w_q.cuda(), q.scales.cuda(), q.biases.cuda())
        args = (C.c_void_p(w.qw.data_ptr()), C.c_void_p(w.sb.data_ptr()), None)
        W = O.Q4Weight(q.w_q.numpy().view(np.uint32), q.scales.float().numpy(),
                       q.biases.float().numpy())
        ref_logits = O.q4_linear64(x.numpy().astype(np.float64), W)  # hi + lo activation
    else:
        wt = (torch.randn((n, k), generator=gen) * 0.02).to(torch.bfloat16)
        w = kernels.DeviceBF16Weight(wt.cuda())
        args = (None, None, C.c_void_p(w.wb.data_ptr()))
        ref_logits = O.linear(x.numpy(), wt.float().numpy(), None, weight_kind="bf16")
    _lib.check(lib.drt_op_lm_head_score(*args, rows, n, k, C.c_void_p(xc.data_ptr()), 0.0, 0, 0,
                                        None, C.c_void_p(scores.data_ptr()),
                                        C.c_void_p(tokens.data_ptr()),
                                        C.c_void_p(logits.data_ptr()), C.c_void_p(ws.data_ptr()),
                                        ws_b, None))
    torch.cuda.synchronize()
    got_logits = logits.cpu().numpy()
    err = np.abs(got_logits - ref_logits).max() / np.abs(ref_logits).max()
    _say(f"  logits err={err:.2e}")
    # q4: fp32 accumulation with the exact-nibble offset trick (~1e-5 of the row max);
    # bf16: the reference rounds logits to bf16, so compare at that resolution
    assert err < (5e-5 if kind == "q4" else 1e-2)
    # scores/tokens must be exactly the float64 scoring of the kernel's own logits
    s_own, t_own = O.raw_max_prob(got_logits)
    assert tokens.cpu().tolist() == t_own
    np.testing.assert_allclose(scores.cpu().numpy(), s_own, rtol=1e-6)


def _q4_dequant64_cuda(w_q, scales, biases):
    """float64 dense weights of q4 rows on the device: nibble i of word j is
    k = 8j + i (low nibble first), w = q * scale + bias per 64-wide group."""
    n, words = w_q.shape
    shifts = torch.arange(8, device=w_q.device, dtype=torch.int32) * 4
    nib = (w_q.unsqueeze(-1) >> shifts) & 15
    q = nib.reshape(n, words * 8 // 64, 64).double()
    return (q * scales.double().unsqueeze(-1) + biases.double().unsqueeze(-1)).reshape(n, -1)


@pytest.mark.parametrize("kind,rows", [("q4", 256), ("q4", 64), ("bf16", 64)])
def test_lm_head_full_vocab_chunked_k3584(kind, rows):
    """Dream's LM head at its real size (vocabulary 152064, K = 3584, every K
    other than 1024): q4 over 256 rows (the large-M GEMM with its statistics
    epilogue, two 128-row tiles) and 64 rows (the chunked kernel, two 32-row
    tiles), bf16 over 64 rows (chunked). Logits against float64 truth computed
    in column chunks (the chunk dequantisation pinned to the oracle's on the
    first chunk), greedy scores and tokens equal to the float64 scoring of the
    device's own logits, and, for q4, the T > 0 sampling rule against the oracle
    on three rows of every 32-row tile."""
    from diffusorrt_amd import _lib, kernels
    from diffusorrt_amd import synthetic as syn
    import ctypes as C

    n, k = 152064, 3584
    _say("lm_head full vocab", kind, rows, n, k)
    gen = torch.Generator().manual_seed(31)
    x = torch.randn((rows, k), generator=gen)
    xc = x.cuda()
    if kind == "q4":
        q = syn.random_q4(gen, n, k)
        w = kernels.DeviceQ4Weight(q.w_q.cuda(), q.scales.cuda(), q.biases.cuda())
        wargs = (C.c_void_p(w.qw.data_ptr()), C.c_void_p(w.sb.data_ptr()), None)
        wq_d, sc_d, bi_d = q.w_q.cuda(), q.scales.cuda(), q.biases.cuda()
        c = 512
        W0 = O.Q4Weight(q.w_q[:c].numpy().view(np.uint32), q.scales[:c].float().numpy(),
                        q.biases[:c].float().numpy())
        dense0 = O.q4_dequant(W0.w_q, W0.scales, W0.biases, dtype=np.float64)
        assert np.array_equal(_q4_dequant64_cuda(wq_d[:c], sc_d[:c], bi_d[:c]).cpu().numpy(),
                              dense0)
        dense = lambda c0, c1: _q4_dequant64_cuda(wq_d[c0:c1], sc_d[c0:c1], bi_d[c0:c1])
    else:
        wt = (torch.randn((n, k), generator=gen) * 0.02).to(torch.bfloat16)
        w = kernels.DeviceBF16Weight(wt.cuda())
        wargs = (None, None, C.c_void_p(w.wb.data_ptr()))
        wt_d = wt.cuda()
        dense = lambda c0, c1: wt_d[c0:c1].double()
    x64 = xc.double()
    ref = torch.empty((rows, n), dtype=torch.float64, device="cuda")
    for c0 in range(0, n, 8192):
        c1 = min(n, c0 + 8192)
        ref[:, c0:c1] = x64 @ dense(c0, c1).T
    if kind == "bf16":  # the reference rounds bf16-weight logits to bf16
        ref = ref.float().to(torch.bfloat16).double()
    lib = _lib.load()
    ws_b = lib.drt_op_lm_head_workspace_bytes(rows, n, k)
    ws = torch.empty(ws_b, dtype=torch.uint8, device="cuda")
    positions = torch.arange(1000, 1000 + rows, dtype=torch.int32, device="cuda")
    for T in ((0.0, 0.7) if kind == "q4" else (0.0,)):
        scores = torch.empty(rows, dtype=torch.float64, device="cuda")
        tokens = torch.empty(rows, dtype=torch.int32, device="cuda")
        logits = torch.empty((rows, n), dtype=torch.float32, device="cuda")
        seed, step = 77, 5
        _lib.check(lib.drt_op_lm_head_score(*wargs, rows, n, k, C.c_void_p(xc.data_ptr()), T,
                                            seed, step, C.c_void_p(positions.data_ptr()),
                                            C.c_void_p(scores.data_ptr()),
                                            C.c_void_p(tokens.data_ptr()),
                                            C.c_void_p(logits.data_ptr()),
                                            C.c_void_p(ws.data_ptr()), ws_b, None))
        torch.cuda.synchronize()
        err = ((logits.double() - ref).abs().amax(dim=1) / ref.abs().amax(dim=1)).max().item()
        _say(f"  T={T} logits rel err max over rows={err:.2e}")
        # q4: fp32 sums over the hi + lo activation (exact-nibble products on
        # the chunked kernel, one fp16 rounding of s * q + b per weight on the
        # GEMM); bf16: compared at the bf16 resolution of the reference's logits
        assert err < (1e-4 if kind == "q4" else 1e-2)
        got = logits.cpu().numpy()
        if T == 0.0:
            s_own, t_own = O.raw_max_prob(got)
            assert tokens.cpu().tolist() == t_own
            np.testing.assert_allclose(scores.cpu().numpy(), s_own, rtol=1e-6)
        else:
            sel = [32 * t + o for t in range(rows // 32) for o in (0, 13, 31)]
            pos = positions.cpu().tolist()
            s_ref, t_ref = O.sampled_max_prob(got[sel], temperature=T, seed=seed, step=step,
                                              positions=[pos[i] for i in sel])
            assert [tokens.cpu().tolist()[i] for i in sel] == t_ref
            np.testing.assert_allclose(scores.cpu().numpy()[sel], s_ref, rtol=1e-6)


@pytest.mark.parametrize("kind,n,k", [("bf16", 2048, 256), ("bf16", 8256, 1024),
                                      ("q4", 8256, 1024)])
def test_lm_head_sampling_matches_oracle_rule(kind, n, k):
    """K = 1024 heads run on the persistent kernel, K = 256 on the chunked one."""
    from diffusorrt_amd import _lib, kernels
    from diffusorrt_amd import synthetic as syn
    import ctypes as C

    rows = 4
    _say("lm_head sampling", kind, rows, n, k)
    gen = torch.Generator().manual_seed(21)
    x = torch.randn((rows, k), generator=gen)
    if kind == "bf16":
        wt = (torch.randn((n, k), generator=gen) * 0.05).to(torch.bfloat16)
        w = kernels.DeviceBF16Weight(wt.cuda())
        wargs = (None, None, C.c_void_p(w.wb.data_ptr()))
    else:
        q = syn.random_q4(gen, n, k)
        w = kernels.DeviceQ4Weight(q.w_q.cuda(), q.scales.cuda(), q.biases.cuda())
        wargs = (C.c_void_p(w.qw.data_ptr()), C.c_void_p(w.sb.data_ptr()), None)
    lib = _lib.load()
    positions = torch.tensor([5, 6, 9, 40], dtype=torch.int32, device="cuda")
    scores = torch.empty(rows, dtype=torch.float64, device="cuda")
    tokens = torch.empty(rows, dtype=torch.int32, device="cuda")
    logits = torch.empty((rows, n), dtype=torch.float32, device="cuda")
    ws_b = lib.drt_op_lm_head_workspace_bytes(rows, n, k)
    ws = torch.empty(ws_b, dtype=torch.uint8, device="cuda")
    xc = x.cuda()
    T, seed, step = 0.7, 1234, 3
    _lib.check(lib.drt_op_lm_head_score(*wargs, rows, n, k,
                                        C.c_void_p(xc.data_ptr()), T, seed, step,
                                        C.c_void_p(positions.data_ptr()),
                                        C.c_void_p(scores.data_ptr()),
                                        C.c_void_p(tokens.data_ptr()),
                                        C.c_void_p(logits.data_ptr()), C.c_void_p(ws.data_ptr()),
                                        ws_b, None))
    torch.cuda.synchronize()
    got_logits = logits.cpu().numpy()
    s_ref, t_ref = O.sampled_max_prob(got_logits, temperature=T, seed=seed, step=step,
                                      positions=positions.cpu().tolist())
    assert tokens.cpu().tolist() == t_ref
    np.testing.assert_allclose(scores.cpu().numpy(), s_ref, rtol=1e-6)
