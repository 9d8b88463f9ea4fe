"""The Python runtime on the GPU: reference-style API behaviour (engine/tests/test_phase30_cuda_qmatvec.py,
test_phase31e_cpu_layers.py) with the HIP library underneath."""
from __future__ import annotations

import random

import numpy as np
import pytest

from conftest import rel_l2
from vinf_3080ti_amd import GGUFTensorType as T
from vinf_3080ti_amd import HIP_MATVEC_TYPES, QUANT_TYPES, synth

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def rt():
    torch = pytest.importorskip("torch")
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    from vinf_3080ti_amd.runtime import HipWeightRuntime

    return HipWeightRuntime()


def test_every_type_matches_cpu_dequant_within_int8_bound(rt, oracle_mod):
    """test_phase31e_cpu_layers.py:29-60: int8-activation matvec vs float64 dequant matvec, bound
    1.05 * sum_g sum|w| * amax_g(x) / 254 + 1e-4 (1 + |ref|) per output."""
    rng = random.Random(3101)
    rows, cols = 12, 512
    for ty in sorted(HIP_MATVEC_TYPES):
        raw = synth.synthetic_rows(ty, rows, cols, np.random.default_rng(rng.getrandbits(32)))
        xs = np.array([[rng.uniform(-1, 1) for _ in range(cols)] for _ in range(3)], np.float32)
        rt.upload_raw("w", raw.tobytes(), ty, cols, rows)
        rt.alloc("w.x", cols * 3)
        rt.alloc("w.y", rows * 3)
        rt.write_floats("w.x", xs.reshape(-1).tolist())
        rt.qmv("w", "w.x", "w.y", 3)
        got = np.array(rt.read_floats("w.y"), np.float64).reshape(3, rows)
        wf = oracle_mod.dequant_rows(int(ty), raw, rows, cols).astype(np.float64)
        for t in range(3):
            ref = wf @ xs[t].astype(np.float64)
            if ty in (T.F32, T.F16):
                bound = np.zeros(rows)
            else:
                amax = np.abs(xs[t].reshape(-1, 32)).max(1)
                bound = (np.abs(wf).reshape(rows, -1, 32).sum(2) * amax / 254.0).sum(1)
            assert np.all(np.abs(got[t] - ref) <= 1.05 * bound + 1e-4 * (1 + np.abs(ref))), ty.name
        rt.free("w")
    assert rt.device_bytes() == 0


def test_matvec_sync_entry(rt, oracle_mod):
    rows, cols = 5, 512
    raw = synth.synthetic_rows(T.Q6_K, rows, cols, 30)
    x = np.random.default_rng(30).uniform(-1, 1, cols).astype(np.float32)
    rt.upload_raw("m", raw.tobytes(), T.Q6_K, cols, rows)
    got = np.array(rt.matvec("m", x.tolist()), np.float32)
    assert rel_l2(got, oracle_mod.qmv(int(T.Q6_K), raw, rows, cols, x, 1)[0]) <= 1e-5
    rt.free("m")


def test_invalid_uploads_and_names_fail_cleanly(rt):
    """test_phase30_cuda_qmatvec.py:127-134 and the error contract of qwen_runtime.cu:1199-1223."""
    with pytest.raises(ValueError):
        rt.upload_raw("w", b"\x00" * 34, 2, 32, 1)  # Q4_0: no matvec
    with pytest.raises(ValueError):
        rt.upload_raw("w", b"\x00" * 33, T.Q8_0, 32, 1)
    with pytest.raises(KeyError):
        rt.matvec("missing", [0.0] * 32)
    rt.upload_raw("q", bytes(34), T.Q8_0, 32, 1)
    rt.alloc("x", 32)
    rt.alloc("y", 1)
    rt.alloc("h", 64, 2)
    with pytest.raises(KeyError):
        rt.qmv("q", "nope", "y")
    with pytest.raises(ValueError):
        rt.qmv("q", "x", "y", 2)  # x too small for 2 tokens
    with pytest.raises(ValueError):
        rt.qmv("q", "x", "y", 0)
    with pytest.raises(TypeError):
        rt.qmv("q", "h", "y")
    with pytest.raises(ValueError):
        rt.argmax_rows("x", 4, 0)
    with pytest.raises(ValueError):
        rt.alloc("z", 0)
    rt.free("q")
    with pytest.raises(KeyError):
        rt.free("q")


def test_buffers_roundtrip_and_argmax(rt):
    rt.alloc("b", 10)
    assert rt.read_floats("b") == [0.0] * 10
    rt.write_floats("b", [1.0, 9.0, 3.0, 9.0], 2)
    assert rt.read_floats("b", 4, 2) == [1.0, 9.0, 3.0, 9.0]
    assert rt.argmax("b", 10) == 3
    assert rt.argmax_rows("b", 5, 2) == [3, 0]
    rt.zero("b")
    assert rt.read_floats("b") == [0.0] * 10


def test_tensor_info_and_reupload(rt):
    raw = synth.synthetic_rows(T.Q4_K, 3, 512, 1)
    rt.upload_raw("t", raw.tobytes(), T.Q4_K, 512, 3)
    addr, ty, rows, cols, rb, nbytes, resident = rt.tensor_info("t")
    assert (ty, rows, cols, rb, nbytes, resident) == (int(T.Q4_K), 3, 512, 288, 864, True)
    assert addr % 256 == 0
    rt.upload_raw("t", raw[:288].tobytes(), T.Q4_K, 512, 1)  # re-upload replaces
    assert rt.tensor_info("t")[2] == 1 and rt.device_bytes() == 288
    rt.free("t")


def test_ntok_above_eight_chunks_like_reference(rt, oracle_mod):
    rows, cols, ntok = 33, 1024, 19
    raw = synth.baseline_rows(T.IQ3_S, rows, cols, 4)
    x = np.random.default_rng(4).standard_normal((ntok, cols)).astype(np.float32)
    rt.upload_raw("c", raw.tobytes(), T.IQ3_S, cols, rows)
    rt.alloc("cx", cols * ntok)
    rt.alloc("cy", rows * ntok)
    rt.write_floats("cx", x.reshape(-1).tolist())
    rt.qmv("c", "cx", "cy", ntok)
    got = np.array(rt.read_floats("cy"), np.float32).reshape(ntok, rows)
    assert rel_l2(got, oracle_mod.qmv(int(T.IQ3_S), raw, rows, cols, x, ntok)) <= 1e-5
    rt.free("c")


def test_wide_inputs_pack_through_the_runtime_workspace(rt, oracle_mod):
    """cols > 24576 takes the pack + packed-matvec path with the runtime's own workspace."""
    rows, cols, ntok = 40, 32768, 3
    raw = synth.baseline_rows(T.Q4_K, rows, cols, 8)
    x = np.random.default_rng(8).standard_normal((ntok, cols)).astype(np.float32)
    rt.upload_raw("wide", raw.tobytes(), T.Q4_K, cols, rows)
    rt.alloc("wx", cols * ntok)
    rt.alloc("wy", rows * ntok)
    rt.write_floats("wx", x.reshape(-1).tolist())
    rt.qmv("wide", "wx", "wy", ntok)
    got = np.array(rt.read_floats("wy"), np.float32).reshape(ntok, rows)
    assert rel_l2(got, oracle_mod.qmv(int(T.Q4_K), raw, rows, cols, x, ntok)) <= 1e-5
    rt.free("wide")


@pytest.mark.parametrize("cols", [5120, 9216])
def test_qmv_group_and_lmhead_argmax(rt, oracle_mod, cols):
    ntok = 2
    rng = np.random.default_rng(cols)
    a = synth.baseline_rows(T.Q5_K, 96, cols, rng)
    b = synth.baseline_rows(T.Q5_K, 40, cols, rng)
    x = rng.standard_normal((ntok, cols)).astype(np.float32)
    rt.upload_raw("ga", a.tobytes(), T.Q5_K, cols, 96)
    rt.upload_raw("gb", b.tobytes(), T.Q5_K, cols, 40)
    rt.alloc("gx", cols * ntok)
    rt.alloc("gya", 96 * ntok)
    rt.alloc("gyb", 40 * ntok)
    rt.write_floats("gx", x.reshape(-1).tolist())
    rt.qmv_group(["ga", "gb"], "gx", ["gya", "gyb"], ntok)
    ya = np.array(rt.read_floats("gya"), np.float32).reshape(ntok, 96)
    yb = np.array(rt.read_floats("gyb"), np.float32).reshape(ntok, 40)
    ra = oracle_mod.qmv(int(T.Q5_K), a, 96, cols, x, ntok)
    rb = oracle_mod.qmv(int(T.Q5_K), b, 40, cols, x, ntok)
    assert rel_l2(ya, ra) <= 1e-5 and rel_l2(yb, rb) <= 1e-5
    ids = rt.lmhead_argmax("ga", "gx", ntok, logits="gya")
    assert ids == rt.argmax_rows("gya", 96, ntok)
    assert ids == rt.lmhead_argmax("ga", "gx", ntok)
    with pytest.raises(ValueError):
        rt.qmv_group(["ga", "t_missing_type"], "gx", ["gya"], ntok)
    with pytest.raises(KeyError):
        rt.qmv_group(["ga", "nope"], "gx", ["gya", "gyb"], ntok)
    # A main type plus Q8_0 small tensors in one group (a gated-delta layer's qkv + beta).
    q8 = synth.baseline_rows(T.Q8_0, 48, cols, rng)
    rt.upload_raw("gq8", q8.tobytes(), T.Q8_0, cols, 48)
    rt.alloc("gyq", 48 * ntok)
    rt.qmv_group(["ga", "gq8"], "gx", ["gya", "gyq"], ntok)
    ya = np.array(rt.read_floats("gya"), np.float32).reshape(ntok, 96)
    yq = np.array(rt.read_floats("gyq"), np.float32).reshape(ntok, 48)
    assert rel_l2(ya, ra) <= 1e-5
    assert rel_l2(yq, oracle_mod.qmv(int(T.Q8_0), q8, 48, cols, x, ntok)) <= 1e-5
    for n in ("ga", "gb", "gq8"):
        rt.free(n)


@pytest.mark.parametrize("ty", [T.Q6_K, T.Q3_K, T.Q4_K, T.Q2_K, T.IQ2_XS, T.IQ3_XXS], ids=lambda t: t.name)
def test_gemm_min_rows_routes_prompts_to_the_mfma_contraction(rt, oracle_mod, ty):
    """Runtime.qmv with ntok >= gemm_min_rows: packed activations and the f16-MFMA prefill contraction (its
    workspace from the runtime), 201 rows (a ragged last row tile) x 70 tokens."""
    rows, cols, ntok = 201, 2048, 70
    raw = synth.baseline_rows(ty, rows, cols, 12)
    x = np.random.default_rng(12).standard_normal((ntok, cols)).astype(np.float32)
    rt.upload_raw("pf", raw.tobytes(), ty, cols, rows)
    rt.alloc("pfx", cols * ntok)
    rt.alloc("pfy", rows * ntok)
    rt.write_floats("pfx", x.reshape(-1).tolist())
    rt.set_gemm_min_rows(64)
    try:
        rt.qmv("pf", "pfx", "pfy", ntok)
    finally:
        rt.set_gemm_min_rows(0)
    got = np.array(rt.read_floats("pfy"), np.float32).reshape(ntok, rows)
    assert rel_l2(got, oracle_mod.qmv(int(ty), raw, rows, cols, x, ntok)) <= 1e-5
    with pytest.raises(ValueError):
        rt.set_gemm_min_rows(-1)
    rt.free("pf")


@pytest.mark.parametrize("ty", [T.Q4_K, T.Q6_K, T.IQ2_XXS, T.Q8_0], ids=lambda t: t.name)
def test_gemm_f16_activations_route(rt, oracle_mod, ty):
    """set_gemm_f16_activations: prompt passes of the f16 path's types through vq_qgemm_f16x_ws (against f16(x)
    times the exact weights); Q8_0 keeps the int8 contraction (against the CPU path)."""
    rows, cols, ntok = 201, 2048, 70
    raw = synth.baseline_rows(ty, rows, cols, 14)
    x = np.random.default_rng(14).standard_normal((ntok, cols)).astype(np.float32)
    rt.upload_raw("pf16", raw.tobytes(), ty, cols, rows)
    rt.alloc("pf16x", cols * ntok)
    rt.alloc("pf16y", rows * ntok)
    rt.write_floats("pf16x", x.reshape(-1).tolist())
    rt.set_gemm_min_rows(64)
    rt.set_gemm_f16_activations(True)
    try:
        rt.qmv("pf16", "pf16x", "pf16y", ntok)
    finally:
        rt.set_gemm_min_rows(0)
        rt.set_gemm_f16_activations(False)
    got = np.array(rt.read_floats("pf16y"), np.float32).reshape(ntok, rows)
    if ty == T.Q8_0:
        ref = oracle_mod.qmv(int(ty), raw, rows, cols, x, ntok)
    else:
        ref = oracle_mod.qgemm_f16x(int(ty), raw, rows, cols, x, ntok)
        # and it is the f16 rounding, not the int8 codes: far from the CPU path at this tolerance
        assert rel_l2(got, oracle_mod.qmv(int(ty), raw, rows, cols, x, ntok)) > 1e-5
    assert rel_l2(got, ref) <= 1e-5
    rt.free("pf16")


def test_upload_gguf_tensor_from_a_file(rt, oracle_mod, tmp_path):
    """upload_gguf_tensor (cuda/qwen_runtime.py:68-86): raw blocks straight from the file's mapping, cols =
    innermost dimension, rows = product of the others, the byte size returned; types without a matvec
    raise UnsupportedModelError."""
    from gguf_writer import write_gguf
    from vinf_3080ti_amd.gguf import GGUFValueType, UnsupportedModelError, load_gguf

    rows, cols = 6, 768
    raw = synth.synthetic_rows(T.Q5_K, rows, cols, 77)
    f32 = np.random.default_rng(78).uniform(-1, 1, (2, 3, 64)).astype(np.float32)
    p = tmp_path / "m.gguf"
    write_gguf(p, [("general.architecture", GGUFValueType.STRING, "qwen35")],
               [("blk.0.attn_q.weight", (cols, rows), T.Q5_K, raw.tobytes()),
                ("stacked", (64, 3, 2), T.F32, f32.tobytes()), ("legacy", (32, 2), T.Q4_0, bytes(36))],
               alignment=64)
    g = load_gguf(p)
    assert rt.upload_gguf_tensor(g, "blk.0.attn_q.weight") == raw.nbytes
    x = np.random.default_rng(79).uniform(-1, 1, cols).astype(np.float32)
    got = np.array(rt.matvec("blk.0.attn_q.weight", x.tolist()), np.float32)
    assert rel_l2(got, oracle_mod.qmv(int(T.Q5_K), raw, rows, cols, x, 1)[0]) <= 1e-5
    assert rt.upload_gguf_tensor(g, "stacked", device_name="s") == f32.nbytes
    assert rt.tensor_info("s")[2:4] == (6, 64)  # rows = 3 * 2, cols = 64
    xs = np.random.default_rng(80).uniform(-1, 1, 64).astype(np.float32)
    got = np.array(rt.matvec("s", xs.tolist()), np.float32)
    assert rel_l2(got, f32.reshape(6, 64).astype(np.float64) @ xs) <= 1e-6
    with pytest.raises(UnsupportedModelError):
        rt.upload_gguf_tensor(g, "legacy")
    with pytest.raises(ValueError):
        rt.upload_gguf_tensor(g, "blk.0.attn_q.weight", group=0)
    rt.free("blk.0.attn_q.weight")
    rt.free("s")


@pytest.mark.parametrize("ntok", [2, 8])
def test_qmv_staged_fuses_silu_mul_norm_and_add(rt, oracle_mod, ntok):
    """Runtime.qmv_staged: v = rmsnorm(silu(x) * x2) * norm, y += W v (the megakernel's QMV flags,
    qwen_megakernel.cu:468-551), against the float64 staged reference within the int8-path bound; the norm
    weights as an uploaded F32 tensor and as a buffer give the same result. 2 tokens stream, 8 take the f16
    small-batch kernel with its RMS prepass."""
    rows, cols = 24, 1024
    rng = np.random.default_rng(91)
    raw = synth.synthetic_rows(T.Q4_K, rows, cols, 91)
    x = rng.standard_normal((ntok, cols)).astype(np.float32)
    x2 = rng.standard_normal((ntok, cols)).astype(np.float32)
    nw = rng.uniform(0.5, 1.5, cols).astype(np.float32)
    y0 = rng.standard_normal((ntok, rows)).astype(np.float32)
    rt.upload_raw("sw", raw.tobytes(), T.Q4_K, cols, rows)
    rt.upload_raw("sw.norm", nw.tobytes(), T.F32, cols, 1)
    for name, n in (("sx", x), ("sx2", x2), ("snw", nw)):
        rt.alloc(name, n.size)
        rt.write_floats(name, n.reshape(-1).tolist())
    outs = []
    for norm in ("sw.norm", "snw"):
        rt.alloc("sy", rows * ntok)
        rt.write_floats("sy", y0.reshape(-1).tolist())
        rt.qmv_staged("sw", "sx", "sy", ntok, x2="sx2", norm=norm, eps=1e-6, add=True)
        outs.append(np.array(rt.read_floats("sy"), np.float64).reshape(ntok, rows))
    assert np.array_equal(outs[0], outs[1])
    v = oracle_mod.stage_x(x, x2, nw, 1e-6, oracle_mod.STAGE_SILU_MUL | oracle_mod.STAGE_NORM)
    wf = oracle_mod.dequant_rows(int(T.Q4_K), raw, rows, cols).astype(np.float64)
    for t in range(ntok):
        ref = wf @ v[t] + y0[t]
        amax = np.abs(v[t].reshape(-1, 32)).max(1)
        bound = (np.abs(wf).reshape(rows, -1, 32).sum(2) * amax / 254.0).sum(1)
        assert np.all(np.abs(outs[0][t] - ref) <= 1.05 * bound + 1e-4 * (1 + np.abs(ref)))
    with pytest.raises(ValueError):
        rt.qmv_staged("sw.norm", "sx", "sy", 1)  # float weights have no staged path
    with pytest.raises(ValueError):
        rt.qmv_staged("sw", "sx", "sy", 1, norm="sw")  # norm must be F32 cols values
    for name in ("sw", "sw.norm"):
        rt.free(name)


def test_norm_and_elementwise_ops(rt, oracle_mod):
    """rmsnorm / gated_rmsnorm / add / silu_mul / sigmoid_mul / copy (qwen_runtime.cu:36-67,1914-1958,
    2200-2218) against the float64 staging restatement (rmsnorm = NORM staging, silu_mul = SILU_MUL staging)
    and scipy's logistic; in-place rmsnorm; deterministic reruns."""
    from scipy.special import expit

    rng = np.random.default_rng(93)
    n, groups = 1000, 3
    x = (rng.standard_normal(n * groups) * 3).astype(np.float32)
    z = rng.standard_normal(n * groups).astype(np.float32)
    w = rng.uniform(0.5, 1.5, n).astype(np.float32)
    rt.upload_raw("nw", w.tobytes(), T.F32, n, 1)
    for name, v in (("ex", x), ("ez", z), ("ey", np.zeros_like(x))):
        rt.alloc(name, v.size)
        rt.write_floats(name, v.tolist())
    rt.rmsnorm("ex", "nw", "ey", n, 1e-6, groups)
    got = np.array(rt.read_floats("ey")).reshape(groups, n)
    ref = oracle_mod.stage_x(x.reshape(groups, n), None, w, 1e-6, oracle_mod.STAGE_NORM)
    assert np.allclose(got, ref, rtol=2e-6, atol=1e-7)
    rt.rmsnorm("ex", "nw", "ey", n, 1e-6, groups)
    assert np.array_equal(np.array(rt.read_floats("ey")).reshape(groups, n), got)
    rt.gated_rmsnorm("ex", "nw", "ez", "ey", n, 1e-6, groups)
    silu_z = oracle_mod.stage_x(z, np.ones_like(z), None, 0.0, oracle_mod.STAGE_SILU_MUL).reshape(groups, n)
    assert np.allclose(np.array(rt.read_floats("ey")).reshape(groups, n), ref * silu_z, rtol=4e-6, atol=1e-7)
    rt.rmsnorm("ex", "nw", "ex", n, 1e-6, groups)  # in place
    assert np.allclose(np.array(rt.read_floats("ex")).reshape(groups, n), ref, rtol=2e-6, atol=1e-7)
    rt.write_floats("ex", x.tolist())
    m = n * groups - 3  # a ragged tail
    rt.add("ex", "ez", "ey", m)
    assert np.array_equal(np.array(rt.read_floats("ey"), np.float32)[:m], (x + z)[:m])
    rt.silu_mul("ex", "ez", "ey", m)
    assert np.allclose(np.array(rt.read_floats("ey"))[:m],
                       oracle_mod.stage_x(x, z, None, 0.0, oracle_mod.STAGE_SILU_MUL)[:m], rtol=2e-6, atol=1e-7)
    rt.sigmoid_mul("ex", "ez", "ey", m)
    assert np.allclose(np.array(rt.read_floats("ey"))[:m], (x.astype(np.float64) * expit(z.astype(np.float64)))[:m],
                       rtol=2e-6, atol=1e-7)
    rt.copy("ey", 10, "ex", 20, 100)
    rt.synchronize()
    assert np.array_equal(np.array(rt.read_floats("ey"), np.float32)[10:110], x[20:120])
    with pytest.raises(ValueError):
        rt.copy("ey", n * groups - 5, "ex", 0, 10)
    with pytest.raises(ValueError):
        rt.copy("ey", -1, "ex", 0, 1)
    with pytest.raises(ValueError):
        rt.rmsnorm("ex", "nw", "ey", n + 1, 1e-6, groups)  # weights hold n values
    with pytest.raises(KeyError):
        rt.add("ex", "nope", "ey", 4)
    rt.free("nw")


def test_split_gated_q_and_rope(rt, oracle_mod):
    """split_gated_q (exact) and NeoX rope (qwen_runtime.cu:70-92) against the float64 rope_neox restatement;
    ntok 3 at a non-zero start position; argument errors as in the reference."""
    rng = np.random.default_rng(95)
    heads, hd, rot, ntok, pos = 4, 32, 16, 3, 1000
    raw = rng.standard_normal(2 * heads * hd).astype(np.float32)
    x = rng.standard_normal(ntok * heads * hd).astype(np.float32)
    for name, v in (("graw", raw), ("gq", np.zeros(heads * hd)), ("gg", np.zeros(heads * hd)), ("rx", x)):
        rt.alloc(name, v.size)
        rt.write_floats(name, np.asarray(v, np.float32).tolist())
    rt.split_gated_q("graw", "gq", "gg", heads, hd)
    r2 = raw.reshape(heads, 2, hd)
    assert np.array_equal(np.array(rt.read_floats("gq"), np.float32), r2[:, 0].reshape(-1))
    assert np.array_equal(np.array(rt.read_floats("gg"), np.float32), r2[:, 1].reshape(-1))
    rt.rope("rx", heads, hd, rot, pos, 1e6, ntok)
    got = np.array(rt.read_floats("rx")).reshape(ntok, heads, hd)
    ref = oracle_mod.rope_neox(x.reshape(ntok, heads, hd), heads, hd, rot, pos, 1e6)
    assert np.allclose(got, ref, rtol=1e-5, atol=2e-6)
    assert np.array_equal(got[..., rot:], x.reshape(ntok, heads, hd)[..., rot:])
    for bad in (dict(rot=15), dict(rot=0), dict(rot=hd + 2), dict(ntok=0)):
        kw = dict(rot=rot, ntok=1) | bad
        with pytest.raises(ValueError):
            rt.rope("rx", heads, hd, kw["rot"], 0, 1e4, kw["ntok"])


@pytest.mark.parametrize("elem", [4, 2])
def test_kv_append_contiguous_caches(rt, elem):
    """kv_append (qwen_runtime.cu:115-128): token t's k/v rows land at position pos + t of each head's
    [max_seq][hd] block (fp16 caches rounded to nearest); other positions keep their contents; errors."""
    rng = np.random.default_rng(97 + elem)
    kvh, hd, max_seq, pos, ntok = 2, 8, 10, 6, 3
    k = rng.standard_normal((ntok, kvh, hd)).astype(np.float32)
    v = rng.standard_normal((ntok, kvh, hd)).astype(np.float32)
    for name, a in (("kk", k), ("kv", v)):
        rt.alloc(name, a.size)
        rt.write_floats(name, a.reshape(-1).tolist())
    for name in ("kc", "vc"):
        rt.alloc(name, kvh * max_seq * hd, elem)
    rt.kv_append("kk", "kv", "kc", "vc", kvh, max_seq, hd, pos, ntok)
    dt = np.float32 if elem == 4 else np.float16
    for name, a in (("kc", k), ("vc", v)):
        got = np.array(rt.read_floats(name), np.float32).reshape(kvh, max_seq, hd)
        want = np.zeros((kvh, max_seq, hd), np.float32)
        want[:, pos:pos + ntok] = a.astype(dt).astype(np.float32).transpose(1, 0, 2)
        assert np.array_equal(got, want), name
    with pytest.raises(ValueError):
        rt.kv_append("kk", "kv", "kc", "vc", kvh, max_seq, hd, max_seq - 2, ntok)
    rt.alloc("vc32" if elem == 2 else "vc16", kvh * max_seq * hd, 4 if elem == 2 else 2)
    with pytest.raises(TypeError):
        rt.kv_append("kk", "kv", "kc", "vc32" if elem == 2 else "vc16", kvh, max_seq, hd, 0, 1)


@pytest.mark.parametrize("elem", [4, 2])
@pytest.mark.parametrize("ntok,seq_len,bidirectional,window", [(1, 300, 0, 0), (3, 77, 0, 0), (4, 129, 1, 0),
                                                               (2, 500, 0, 64), (1, 1, 0, 0)])
def test_attention_matches_oracle(rt, oracle_mod, elem, ntok, seq_len, bidirectional, window):
    """attention (qwen_runtime.cu:128-162) vs the float64 restatement: GQA 8 heads over 2 kv heads, hd 128,
    causal / bidirectional / sliding window, fp32 and fp16 caches (the cache values as stored)."""
    rng = np.random.default_rng(1000 + 7 * ntok + seq_len + elem)
    heads, kvh, hd, max_seq = 8, 2, 128, 520
    q = rng.standard_normal((ntok, heads, hd)).astype(np.float32)
    dt = np.float32 if elem == 4 else np.float16
    kc = (rng.standard_normal((kvh, max_seq, hd)) * 0.3).astype(dt)
    vc = rng.standard_normal((kvh, max_seq, hd)).astype(dt)
    rt.alloc("aq", q.size)
    rt.write_floats("aq", q.reshape(-1).tolist())
    rt.alloc("ao", q.size)
    for name, a in (("akc", kc), ("avc", vc)):
        rt.alloc(name, a.size, elem)
        rt.write(name, a.tobytes())
    rt.attention("aq", "akc", "avc", "ao", heads, kvh, hd, max_seq, seq_len, ntok, bidirectional, window)
    got = np.array(rt.read_floats("ao")).reshape(ntok, heads, hd)
    ref = oracle_mod.attention(q, kc, vc, heads, kvh, seq_len, bool(bidirectional), window)
    assert np.allclose(got, ref, rtol=2e-5, atol=2e-5)
    with pytest.raises(ValueError):
        rt.attention("aq", "akc", "avc", "ao", heads, 3, hd, max_seq, seq_len, ntok)
    with pytest.raises(ValueError):
        rt.attention("aq", "akc", "avc", "ao", heads, kvh, hd, max_seq, max_seq, 2)


def test_conv_update_matches_oracle(rt, oracle_mod):
    """conv_update (qwen_runtime.cu:401-426): outputs, final state and per-token snapshots vs the float64
    restatement; K = 4 over 3 tokens, then one more token continuing from the updated state."""
    rng = np.random.default_rng(99)
    ch, K, ntok = 300, 4, 3
    x = rng.standard_normal((ntok + 1, ch)).astype(np.float32)
    s0 = rng.standard_normal((ch, K)).astype(np.float32)
    w = (rng.standard_normal((ch, K)) * 0.5).astype(np.float32)
    rt.upload_raw("cw", w.tobytes(), T.F32, K, ch)
    for name, a in (("cx", x[:ntok]), ("cs", s0), ("co", np.zeros((ntok, ch))), ("csn", np.zeros((ntok - 1, ch, K))),
                    ("cx1", x[ntok:])):
        rt.alloc(name, a.size)
        rt.write_floats(name, np.asarray(a, np.float32).reshape(-1).tolist())
    rt.conv_update("cx", "cs", "cw", "co", ch, K, ntok, "csn")
    out, st, snaps = oracle_mod.conv_update(x[:ntok], s0, w)
    assert np.allclose(np.array(rt.read_floats("co")).reshape(ntok, ch), out, rtol=1e-5, atol=1e-6)
    assert np.allclose(np.array(rt.read_floats("cs")).reshape(ch, K), st, rtol=0, atol=0)
    assert np.allclose(np.array(rt.read_floats("csn")).reshape(ntok - 1, ch, K), snaps, rtol=0, atol=0)
    rt.conv_update("cx1", "cs", "cw", "co", ch, K, 1)
    out2, _, _ = oracle_mod.conv_update(x[ntok:], st, w)
    assert np.allclose(np.array(rt.read_floats("co"))[:ch], out2[0], rtol=1e-5, atol=1e-6)
    with pytest.raises(ValueError):
        rt.conv_update("cx", "cs", "cw", "co", ch, K, 0)
    rt.free("cw")


@pytest.mark.parametrize("head_order", [0, 1])
def test_gated_delta_matches_oracle(rt, oracle_mod, head_order):
    """gated_delta (qwen_runtime.cu:515-567): 3 tokens, 2 key heads over 4 value heads, kd 128, vd 96;
    outputs, final state and snapshots vs the float64 restatement."""
    rng = np.random.default_rng(101 + head_order)
    kh, vh, kd, vd, ntok = 2, 4, 128, 96, 3
    cdim = 2 * kh * kd + vh * vd
    conv = rng.standard_normal((ntok, cdim)).astype(np.float32)
    b = rng.standard_normal((ntok, vh)).astype(np.float32)
    a = rng.standard_normal((ntok, vh)).astype(np.float32)
    ssm_a = -rng.uniform(0.1, 2.0, vh).astype(np.float32)
    dt = rng.standard_normal(vh).astype(np.float32)
    s0 = (rng.standard_normal((vh, kd, vd)) * 0.1).astype(np.float32)
    rt.upload_raw("gda", ssm_a.tobytes(), T.F32, vh, 1)
    rt.upload_raw("gdt", dt.tobytes(), T.F32, vh, 1)
    for name, arr in (("gc", conv), ("gb", b), ("ga", a), ("gs", s0), ("go", np.zeros((ntok, vh, vd))),
                      ("gsn", np.zeros((ntok - 1, vh, kd, vd)))):
        rt.alloc(name, arr.size)
        rt.write_floats(name, np.asarray(arr, np.float32).reshape(-1).tolist())
    rt.gated_delta("gc", "gb", "ga", "gda", "gdt", "gs", "go", kh, vh, kd, vd, 1e-6, head_order, ntok, "gsn")
    out, S, snaps = oracle_mod.gated_delta(conv, b, a, ssm_a, dt, s0, kh, vh, kd, vd, 1e-6, head_order)
    assert np.allclose(np.array(rt.read_floats("go")).reshape(ntok, vh, vd), out, rtol=1e-4, atol=2e-5)
    assert np.allclose(np.array(rt.read_floats("gs")).reshape(vh, kd, vd), S, rtol=1e-4, atol=2e-5)
    assert np.allclose(np.array(rt.read_floats("gsn")).reshape(ntok - 1, vh, kd, vd), snaps, rtol=1e-4, atol=2e-5)
    with pytest.raises(ValueError):
        rt.gated_delta("gc", "gb", "ga", "gda", "gdt", "gs", "go", 3, vh, kd, vd, 1e-6, head_order, ntok)
    rt.free("gda")
    rt.free("gdt")


def test_executor_load_path_with_arena_groups_and_stream_order(oracle_mod):
    """The calls QwenGpuExecutor._load_weights makes on an all-resident model (src/vinf/qwen_gpu.py:575-630):
    weight groups, the arena, uploads into each, the stream order, and the byte counters of :673,833,1263
    (qwen_runtime.cu:1436-1811). Every tensor must still multiply correctly from wherever it was carved."""
    torch = pytest.importorskip("torch")
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    from vinf_3080ti_amd.runtime import HipWeightRuntime

    rt = HipWeightRuntime()
    rows, cols = 40, 512
    rng = np.random.default_rng(604)
    mats = {n: (ty, synth.synthetic_rows(ty, rows, cols, rng)) for n, ty in
            (("g.a", T.Q4_K), ("g.b", T.Q6_K), ("s.a", T.Q3_K), ("s.b", T.Q8_0), ("p.a", T.IQ4_XS))}
    padded = {n: (w.nbytes + 16 + 255) // 256 * 256 for n, (_, w) in mats.items()}
    gran = rt.vmm_granularity()
    with pytest.raises(RuntimeError):
        rt.add_weight_group(gran)  # before set_weight_space
    rt.set_weight_space(2 * gran)
    gid = rt.add_weight_group(padded["g.a"] + padded["g.b"])
    with pytest.raises(ValueError):
        rt.add_weight_group(2 * gran)  # exhausted
    rt.set_arena(padded["s.a"])  # room for s.a only: s.b falls back to its own allocation
    for n in ("g.a", "g.b"):
        rt.upload(n, mats[n][1].tobytes(), int(mats[n][0]), cols, rows, True, gid)
    for n in ("s.a", "s.b"):
        rt.upload_raw(n, mats[n][1].tobytes(), mats[n][0], cols, rows)
    rt.upload_raw("p.a", mats["p.a"][1].tobytes(), T.IQ4_XS, cols, rows, resident=False)
    big = synth.synthetic_rows(T.Q8_0, 4096, cols, rng)  # 2.2 MB: more than the rest of the 2 MiB group
    with pytest.raises(ValueError):
        rt.upload("g.c", big.tobytes(), int(T.Q8_0), cols, 4096, True, gid)  # group full
    with pytest.raises(ValueError):
        rt.upload("g.c", mats["g.a"][1].tobytes(), int(T.Q4_K), cols, rows, True, gid + 1)  # unknown group
    with pytest.raises(RuntimeError):
        rt.set_arena(1 << 20)  # s.a lives in it

    x = rng.standard_normal((2, cols)).astype(np.float32)
    rt.alloc("x", 2 * cols)
    rt.alloc("y", 2 * rows)
    rt.write_floats("x", x.reshape(-1))
    for n, (ty, w) in mats.items():
        rt.qmv(n, "x", "y", 2)
        got = np.array(rt.read_floats("y"), np.float32).reshape(2, rows)
        assert rel_l2(got, oracle_mod.qmv(int(ty), w, rows, cols, x, 2)) <= 1e-5, n

    rt.set_stream_order(["p.a"], 3)
    rt.set_stream_order([], 0)
    with pytest.raises(ValueError):
        rt.set_stream_order(["s.a"], 3)  # resident tensors do not stream
    with pytest.raises(ValueError):
        rt.set_stream_order(["p.a", "p.a"], 3)
    with pytest.raises(ValueError):
        rt.set_stream_order(["nope"], 3)
    rt.reserve_ring(1 << 20, 3)

    groups = rt.weight_groups()
    assert groups == [(gran, True, ["g.a", "g.b"])]
    assert rt.promote_group(gid) is True
    with pytest.raises(RuntimeError):
        rt.demote_group(gid)
    with pytest.raises(ValueError):
        rt.promote_group(gid + 1)
    assert rt.staging_bytes() == rt.pinned_bytes() == rt.streamed_bytes() == 0
    assert rt.buffer_bytes() == 4 * (2 * cols + 2 * rows)
    own = padded["s.b"] + padded["p.a"]
    assert rt.vram_bytes() >= gran + padded["s.a"] + own + rt.buffer_bytes()
    assert rt.device_bytes() == sum(w.nbytes for _, w in mats.values())

    rt.alloc("kv", 4096, 2, True)  # a "virtual" buffer is backed in full
    assert rt.map_cost("kv", 0, 4096) == 0
    assert rt.map_range("kv", 1024, 1024) is True
    rt.unmap_range("kv", 1024, 1024)
    with pytest.raises(ValueError):
        rt.map_range("kv", 4000, 200)
    for n in mats:
        rt.free(n)
    rt.set_arena(0)
