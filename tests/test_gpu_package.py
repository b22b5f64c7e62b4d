"""Package loading on the device: the HIP quantizer and bf16 cast bit-exact against
the oracle, and runtimes opened from package directories against the oracle's
forward on the same prepared weights."""
from __future__ import annotations


import numpy as np
import pytest

from oracle import forward as F
from oracle import ops as O

from helpers import LOGITS_REL_TOL, rel_err_rows, tiny_dream_geometry, tiny_geometry
from package_writer import random_weights, write_package

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu


def _say(*a):
    print("[case]", *a, flush=True)


def _quantize_on_device(w: torch.Tensor):
    from diffusorrt_amd import _lib

    lib = _lib.load()
    n, k = w.shape
    src = w.contiguous().cuda()
    w_q = torch.empty((n, k // 8), dtype=torch.int32, device="cuda")
    s = torch.empty((n, k // 64), dtype=torch.bfloat16, device="cuda")
    b = torch.empty((n, k // 64), dtype=torch.bfloat16, device="cuda")
    code = _lib.F32 if w.dtype == torch.float32 else _lib.BF16
    _lib.check(lib.drt_op_q4_quantize(src.data_ptr(), code, n, k, w_q.data_ptr(), s.data_ptr(),
                                      b.data_ptr(), None))
    torch.cuda.synchronize()
    return (w_q.cpu().numpy().view(np.uint32), s.cpu().view(torch.int16).numpy().view(np.uint16),
            b.cpu().view(torch.int16).numpy().view(np.uint16))


def _special_groups(n_rows: int, k: int) -> np.ndarray:
    """Rows of groups the quantizer treats specially: zero, constant, exact ramps
    of both orientations, a .5 tie, tiny and large magnitudes, one-signed."""
    rng = np.random.default_rng(7)
    w = rng.normal(0, 0.02, (n_rows, k)).astype(np.float32)
    ramp = np.arange(64) % 16
    w[0, :64] = 0.0
    w[0, 64:128] = 0.3
    w[1, :64] = -1.0 + 0.125 * ramp
    w[1, 64:128] = 1.0 - 0.125 * ramp
    w[2, :64] = -1.0 + 0.125 * ramp
    w[2, 2] = -0.6875  # q = 2.5 exactly
    w[3, :64] = rng.normal(0, 1e-30, 64)
    w[3, 64:128] = rng.normal(0, 300.0, 64)
    w[4, :64] = np.abs(w[4, :64])
    w[4, 64:128] = -np.abs(w[4, 64:128])
    return w


@pytest.mark.parametrize("n,k,dtype", [(64, 1024, "bf16"), (96, 3072, "f32"), (32, 128, "f32"),
                                       (128, 18944, "bf16")])
def test_q4_quantize_bit_exact(n, k, dtype):
    _say("q4_quantize", n, k, dtype)
    w = _special_groups(n, k)
    t = torch.from_numpy(w)
    if dtype == "bf16":
        t = t.to(torch.bfloat16)
    got_q, got_s, got_b = _quantize_on_device(t)
    ref_q, ref_s, ref_b = O.q4_quantize(t.float().numpy())
    assert np.array_equal(got_q, ref_q), np.argwhere(got_q != ref_q)[:5]
    assert np.array_equal(got_s, O.bf16_bits(ref_s))
    assert np.array_equal(got_b, O.bf16_bits(ref_b))
    assert O.q4_unpack(got_q)[2, 2] == 3  # the tie, halves away from zero


def test_q4_quantize_refuses_indivisible_k():
    from diffusorrt_amd import _lib

    lib = _lib.load()
    buf = torch.empty(4096, dtype=torch.bfloat16, device="cuda")
    status = lib.drt_op_q4_quantize(buf.data_ptr(), _lib.BF16, 32, 96, buf.data_ptr(),
                                    buf.data_ptr(), buf.data_ptr(), None)
    assert status == _lib.UNSUPPORTED


def test_cast_bf16_bit_exact():
    from diffusorrt_amd import _lib

    lib = _lib.load()
    x = np.random.default_rng(8).normal(0, 3, 100_003).astype(np.float32)
    x[:6] = [0.0, -0.0, 1.0 + 2**-8, 1.0 + 3 * 2**-8, 3.4e38, -1e-40]
    src = torch.from_numpy(x).cuda()
    out = torch.empty(x.size, dtype=torch.bfloat16, device="cuda")
    _lib.check(lib.drt_op_cast_bf16(src.data_ptr(), out.data_ptr(), x.size, None))
    torch.cuda.synchronize()
    got = out.cpu().view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(got, O.bf16_bits(x))


def _oracle_weights(host: dict, q4: bool) -> dict:
    from diffusorrt_amd.package import is_quantized_linear

    W = {}
    for name, t in host.items():
        a = t.float().numpy()
        W[name] = O.Q4Weight(*O.q4_quantize(a)) if q4 and is_quantized_linear(name) else \
            O.bf16_round(a)
    return W


@pytest.mark.parametrize("fmt,q4,dream", [("safetensors", True, False), ("npz", True, False),
                                          ("safetensors", False, False), ("npz", True, True)])
def test_runtime_from_package_matches_oracle(tmp_path, fmt, q4, dream):
    from diffusorrt_amd import synthetic as syn
    from diffusorrt_amd.package import load_package
    from diffusorrt_amd.runtime import Runtime, bd3_session_config, fixed_quota_session_config

    _say("package runtime", fmt, "q4" if q4 else "bf16", "dream" if dream else "bd3")
    g = tiny_dream_geometry() if dream else tiny_geometry()
    host = random_weights(g, seed=21, dtype=torch.bfloat16 if fmt == "safetensors" else torch.float32)
    root = write_package(tmp_path / "pkg", g, host, fmt=fmt, max_shard_bytes=400_000)
    ec = {"linear_quant_bits": 4, "linear_quant_group_size": 64} if q4 else {}
    W = _oracle_weights(host, q4)
    cfg = syn.oracle_config(g, "q4" if q4 else "bf16")
    if q4:  # the device-prepared bundles are the oracle's, bit for bit
        pm = load_package(root, linear_quant_bits=4)
        for name, v in pm.weights.items():
            if isinstance(v, syn.Q4Tensor):
                assert np.array_equal(v.w_q.cpu().numpy().view(np.uint32), W[name].w_q), name
                assert np.array_equal(v.scales.float().cpu().numpy(), W[name].scales), name
                assert np.array_equal(v.biases.float().cpu().numpy(), W[name].biases), name
            else:
                assert np.array_equal(v.float().cpu().numpy(), W[name]), name
        del pm
    rt = Runtime(str(root), engine_config=ec, max_forward_rows=512, max_positions=1024)
    assert rt.weight_kind == ("q4" if q4 else "bf16")
    rng = np.random.default_rng(3)
    if dream:
        x = rng.integers(0, 900, 64).tolist() + [g.mask_token_id] * 64
        scope = list(range(64, 128))
        with rt.session(fixed_quota_session_config(256, 16, len(x))) as s:
            got = s.execute_window(x, scope).array()
        ref = F.window_logits(W, cfg, x, scope, mask_kind="bidirectional", mask_geometry=None,
                              logits_convention="dream_ar_shift")
    else:
        x = rng.integers(0, 900, 64).tolist() + [g.mask_token_id] * 32
        scope = list(range(64, 96))
        with rt.session(bd3_session_config(32, 16, len(x))) as s:
            got = s.execute_window(x, scope, mask_geometry=(0, 32)).array()
        ref = F.forward_full(W, cfg, x, mask_kind="d2f_hybrid", mask_geometry=(0, 32),
                             output_rows=scope)
    err = rel_err_rows(got, ref)
    _say(f"  logits rel err max={err.max():.2e}")
    assert err.max() < LOGITS_REL_TOL
    rt.close()


def test_engine_generates_from_package(tmp_path):
    from diffusorrt_amd import decode
    from diffusorrt_amd.engine import RocmEngine
    from diffusorrt_amd.runtime import bd3_session_config

    _say("engine from package")
    g = tiny_geometry()
    root = write_package(tmp_path / "pkg", g, random_weights(g, 22, dtype=torch.bfloat16))
    prompt = np.random.default_rng(4).integers(0, 900, 64).tolist()
    with RocmEngine(str(root), precision="q4", max_forward_rows=512, max_positions=256) as eng:
        assert eng.plan.decode_strategy == "bd3_fixed_quota" and eng.runtime.weight_kind == "q4"
        res = eng.generate_ids(prompt, max_tokens=64)
        assert res.backend == "rocm" and res.decodes == 1 and res.steps == 128
        # the engine is the session API plus its plan: the same tokens either way
        with eng.runtime.session(bd3_session_config(32, res.steps, 128)) as s:
            direct = decode.generate_device_tokens(
                s, prompt, max_tokens=64, mask_token_id=g.mask_token_id,
                eos_token_id=g.eos_token_id, steps=res.steps, block_size=32)
        assert res.token_ids == direct.visible_generated_token_ids
        # seeded sampling on the device is reproducible
        a = eng.generate_ids(prompt, max_tokens=32, temperature=0.8, seed=7)
        b = eng.generate_ids(prompt, max_tokens=32, temperature=0.8, seed=7)
        assert a.seed == 7 and a.token_ids == b.token_ids
        # no limit: one decode up to the sequence limit (256 - 64 positions)
        c = eng.generate_ids(prompt, max_tokens=None)
        assert c.decodes == 1 and c.budget == 192 and len(c.token_ids) <= 192


def test_engine_dream_block_threshold_from_package(tmp_path):
    from diffusorrt_amd import decode
    from diffusorrt_amd.engine import RocmEngine
    from diffusorrt_amd.runtime import block_threshold_session_config

    _say("engine dream block_threshold from package")
    g = tiny_dream_geometry()
    root = write_package(tmp_path / "pkg", g, random_weights(g, 23, dtype=torch.bfloat16))
    prompt = np.random.default_rng(6).integers(0, 900, 45).tolist()
    with RocmEngine(str(root), precision="q4", max_forward_rows=512, max_positions=256) as eng:
        assert eng.plan.decode_strategy == "block_threshold" and eng.plan.block_size == 8
        res = eng.generate_ids(prompt, max_tokens=16)
        assert res.decodes == 1 and res.committed_token_count == 16
        with eng.runtime.session(block_threshold_session_config(8, 512, 61)) as s:
            direct = decode.generate_device_tokens(
                s, prompt, max_tokens=16, mask_token_id=g.mask_token_id,
                eos_token_id=g.eos_token_id, steps=512, block_size=8,
                decode_strategy="block_threshold")
        assert res.token_ids == direct.visible_generated_token_ids


def _device_bundles_as_oracle(root, host: dict, sample_rows: int = 96) -> dict:
    """The device-prepared weights of a package as oracle weights, each q4 linear
    first checked bit-exact against the oracle's quantizer on its first and last
    ``sample_rows`` rows (and every other tensor in full): quantizing whole 7B
    layers in numpy would take minutes, the device does it in milliseconds."""
    from diffusorrt_amd import synthetic as syn
    from diffusorrt_amd.package import load_package

    pm = load_package(root, linear_quant_bits=4)
    W = {}
    for name, v in pm.weights.items():
        a = host[name].float().numpy()
        if isinstance(v, syn.Q4Tensor):
            got = (v.w_q.cpu().numpy().view(np.uint32), v.scales.float().cpu().numpy(),
                   v.biases.float().cpu().numpy())
            n = a.shape[0]
            for rows in (slice(0, min(sample_rows, n)), slice(max(0, n - sample_rows), n)):
                ref = O.q4_quantize(a[rows])
                for g_, r_ in zip(got, ref):
                    assert np.array_equal(g_[rows], r_), name
            W[name] = O.Q4Weight(*got)
        else:
            got = v.float().cpu().numpy()
            assert np.array_equal(got, O.bf16_round(a)), name
            W[name] = got
    del pm
    return W


@pytest.mark.timeout(400)
@pytest.mark.parametrize("dream", [False, True])
def test_real_shape_package_matches_oracle(tmp_path, dream):
    """A package with the real BD3 (Qwen3-0.6B) or Dream (Qwen2.5-7B: q/k/v
    biases, untied head, 28 / 4 heads) layer shapes, two layers and a 4096-token
    vocabulary, written as bf16 safetensors and quantized on the device, against
    the oracle's forward. BD3: the oracle quantizes every weight itself. Dream:
    the oracle takes the device-quantized weights after checking them bit-exact
    against its quantizer on a row sample of every linear (the whole 7B layers
    would take minutes in numpy)."""
    import dataclasses

    from diffusorrt_amd import synthetic as syn
    from diffusorrt_amd.runtime import Runtime, bd3_session_config, fixed_quota_session_config

    _say("real-shape package", "dream" if dream else "bd3")
    base = syn.DREAM_QWEN25_7B if dream else syn.BD3_QWEN3_06B
    g = dataclasses.replace(base, layer_count=2, vocab_size=4096, mask_token_id=4000,
                            eos_token_id=4001, max_position_embeddings=4096)
    host = random_weights(g, seed=31, dtype=torch.bfloat16)
    root = write_package(tmp_path / "pkg", g, host, max_shard_bytes=64 << 20)
    W = _device_bundles_as_oracle(root, host) if dream else _oracle_weights(host, q4=True)
    del host
    cfg = syn.oracle_config(g, "q4")
    rt = Runtime(str(root), engine_config={"linear_quant_bits": 4}, max_forward_rows=512,
                 max_positions=1024)
    rng = np.random.default_rng(8)
    if dream:
        x = rng.integers(0, 3900, 32).tolist() + [g.mask_token_id] * 32
        scope = list(range(32, 64))
        with rt.session(fixed_quota_session_config(256, 8, len(x))) as s:
            got = s.execute_window(x, scope).array()
        ref = F.window_logits(W, cfg, x, scope, mask_kind="bidirectional", mask_geometry=None,
                              logits_convention="dream_ar_shift")
    else:
        x = rng.integers(0, 3900, 64).tolist() + [g.mask_token_id] * 32
        scope = list(range(64, 96))
        with rt.session(bd3_session_config(32, 8, len(x))) as s:
            got = s.execute_window(x, scope, mask_geometry=(0, 32)).array()
        ref = F.forward_full(W, cfg, x, mask_kind="d2f_hybrid", mask_geometry=(0, 32),
                             output_rows=scope)
    err = rel_err_rows(got, ref)
    _say(f"  logits rel err max={err.max():.2e}")
    assert err.max() < LOGITS_REL_TOL
    rt.close()
