"""GPU parity of the HIP path against the oracle and the reference's golden vectors, through the C ABI.

Bars: quantizer, dequantization and integer partials bit-exact; fp32 outputs within rel-L2 <= 1e-5 of
the reference CPU path (the oracle is bit-identical to it, see test_oracle.py).
"""
from __future__ import annotations

import ctypes

import numpy as np
import pytest

from conftest import rel_l2
from vinf_3080ti_amd import GGUFTensorType as T
from vinf_3080ti_amd import QUANT_TYPES, synth

pytestmark = pytest.mark.gpu
ALL_TYPES = list(QUANT_TYPES) + [T.F32, T.F16]
REL_L2_TOL = 1e-5  # north-star fp32 tolerance vs the reference CPU path


@pytest.fixture(scope="module")
def env():
    torch = pytest.importorskip("torch")
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    from vinf_3080ti_amd import _lib

    lib = _lib.load()
    assert lib.vq_init() == 0
    return torch, lib


def dev(torch, a: np.ndarray):
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def wdev(torch, w: np.ndarray):
    """Weights with the 16-byte tail pad the kernels may read."""
    buf = np.zeros(w.size + 256, np.uint8)
    buf[: w.size] = w
    return dev(torch, buf)


def P(t) -> int:
    return t.data_ptr()


def pack_ref(q: np.ndarray, d: np.ndarray, stride: int) -> np.ndarray:
    """Expected packed activation records: q int8 | d fp32 | (sum q[0:16], sum q[16:32]) as int16 pairs, zero pad."""
    ntok, cols = q.shape
    ng = cols // 32
    out = np.zeros((ntok, stride), np.uint8)
    out[:, :cols] = q.view(np.uint8)
    out[:, cols : cols + 4 * ng] = np.ascontiguousarray(d, dtype=np.float32).view(np.uint8)
    h = q.reshape(ntok, ng, 2, 16).astype(np.int64).sum(-1).astype(np.int16)  # [t][g][half]: low, high
    out[:, cols + 4 * ng : cols + 8 * ng] = np.ascontiguousarray(h).view(np.uint8).reshape(ntok, 4 * ng)
    return out.reshape(-1)


def gpu_qmv(torch, lib, ty, w, rows, cols, x, ntok, fast=False):
    """vq_qmv with the minimal workspace (streaming matvec), or with vq_qmv_workspace_bytes_for (fast: the
    MFMA small-batch path for 2..16 tokens)."""
    wd, xd = wdev(torch, w), dev(torch, x.astype(np.float32).reshape(ntok, cols))
    y = torch.empty(ntok, rows, dtype=torch.float32, device="cuda")
    nws = (lib.vq_qmv_workspace_bytes_for(int(ty), rows, cols, ntok) if fast
           else lib.vq_qmv_workspace_bytes(cols, ntok))
    ws = torch.empty(max(nws, 1), dtype=torch.uint8, device="cuda")
    st = lib.vq_qmv(int(ty), P(wd), rows, cols, P(xd), ntok, P(y), P(ws), nws, None)
    assert st == 0, lib.vq_status_string(st)
    torch.cuda.synchronize()
    return y.cpu().numpy()


@pytest.mark.parametrize("ntok,cols", [(1, 256), (3, 1024), (8, 5120), (2, 17408)])
def test_quantize_x_bit_exact(env, oracle_mod, ntok, cols):
    torch, lib = env
    rng = np.random.default_rng(cols + ntok)
    x = (rng.standard_normal((ntok, cols)) * rng.choice([1e-3, 1.0, 30.0], size=(ntok, cols))).astype(np.float32)
    x[0, :32] = 0.0  # a zero group
    x[-1, 64:96] = np.float32(0.5) * np.arange(-16, 16, dtype=np.float32)  # exact halves after scaling
    xd_ = dev(torch, x)
    ng = cols // 32
    xq = torch.empty(ntok, cols, dtype=torch.int8, device="cuda")
    d = torch.empty(ntok, ng, dtype=torch.float32, device="cuda")
    s = torch.empty(ntok, ng, dtype=torch.float32, device="cuda")
    assert lib.vq_quantize_x(P(xd_), ntok, cols, P(xq), P(d), P(s), None) == 0
    stride = lib.vq_xpack_bytes(cols, 1)
    xp = torch.full((lib.vq_xpack_bytes(cols, ntok),), 0xAB, dtype=torch.uint8, device="cuda")
    assert lib.vq_pack_x(P(xd_), ntok, cols, P(xp), None) == 0
    torch.cuda.synchronize()
    q_ref, d_ref, s_ref = oracle_mod.quantize_x(x, ntok, cols)
    assert np.array_equal(xq.cpu().numpy(), q_ref)
    assert np.array_equal(d.cpu().numpy().view(np.uint32), d_ref.view(np.uint32))
    assert np.array_equal(s.cpu().numpy().view(np.uint32), s_ref.view(np.uint32))
    assert np.array_equal(xp.cpu().numpy(), pack_ref(q_ref, d_ref, stride))


@pytest.mark.parametrize("ty", ALL_TYPES, ids=lambda t: t.name)
def test_dequant_bit_exact(env, oracle_mod, ty):
    torch, lib = env
    rows, cols = 7, 1024
    w = synth.baseline_rows(ty, rows, cols, 11 + int(ty))
    out = torch.empty(rows, cols, dtype=torch.float32, device="cuda")
    wd = wdev(torch, w)
    assert lib.vq_dequant_rows(int(ty), P(wd), rows, cols, P(out), None) == 0
    torch.cuda.synchronize()
    ref = oracle_mod.dequant_rows(int(ty), w, rows, cols)
    assert np.array_equal(out.cpu().numpy().view(np.uint32), ref.view(np.uint32))


@pytest.mark.parametrize("ty", QUANT_TYPES, ids=lambda t: t.name)
def test_int_partials_bit_exact(env, oracle_mod, ty):
    torch, lib = env
    rows, cols, ntok = 9, 1024, 3
    rng = np.random.default_rng(40 + int(ty))
    w = synth.baseline_rows(ty, rows, cols, rng)
    x = rng.standard_normal((ntok, cols)).astype(np.float32)
    xq, xd, _ = oracle_mod.quantize_x(x, ntok, cols)
    part = torch.empty(ntok, rows, cols // 32, 2, dtype=torch.int32, device="cuda")
    wd, xpd = wdev(torch, w), dev(torch, pack_ref(xq, xd, lib.vq_xpack_bytes(cols, 1)))
    assert lib.vq_int_partials(int(ty), P(wd), rows, cols, P(xpd), ntok, P(part), None) == 0
    torch.cuda.synchronize()
    assert np.array_equal(part.cpu().numpy(), oracle_mod.int_partials(int(ty), w, rows, cols, xq, ntok))


@pytest.mark.parametrize("ty", ALL_TYPES, ids=lambda t: t.name)
def test_qmv_matches_reference_golden(env, golden, ty):
    torch, lib = env
    w, x, y = golden[f"w_{ty.name}"], golden[f"x_{ty.name}"], golden[f"y_{ty.name}"]
    got = gpu_qmv(torch, lib, ty, w, y.shape[1], x.shape[1], x, x.shape[0])
    assert rel_l2(got, y) <= REL_L2_TOL


@pytest.mark.parametrize("ty", ALL_TYPES, ids=lambda t: t.name)
@pytest.mark.parametrize("ntok", [1, 2, 5, 8, 11])
def test_qmv_matches_oracle(env, oracle_mod, ty, ntok):
    torch, lib = env
    rows, cols = 37, 2048 if ty not in (T.F32, T.F16) else 1024
    rng = np.random.default_rng(1000 * ntok + int(ty))
    w = synth.baseline_rows(ty, rows, cols, rng)
    x = rng.standard_normal((ntok, cols)).astype(np.float32)
    got = gpu_qmv(torch, lib, ty, w, rows, cols, x, ntok)
    ref = oracle_mod.qmv(int(ty), w, rows, cols, x, ntok)
    for t in range(ntok):
        assert rel_l2(got[t], ref[t]) <= REL_L2_TOL, (ty.name, ntok, t)


@pytest.mark.parametrize("ty", [T.Q4_K, T.Q3_K, T.Q6_K, T.Q8_0, T.IQ2_XXS, T.F16], ids=lambda t: t.name)
@pytest.mark.parametrize("ntok", [17, 40])
@pytest.mark.parametrize("fast", [False, True], ids=["min_ws", "full_ws"])
def test_qmv_more_tokens_than_a_pass(env, oracle_mod, ty, ntok, fast):
    """vq_qmv beyond 16 tokens (more than one streaming pass or small-batch tile), with the minimal workspace and
    with vq_qmv_workspace_bytes_for: every token within the fp32 bar of the CPU path."""
    torch, lib = env
    rows, cols = 70, 1024
    rng = np.random.default_rng(31 * ntok + int(ty))
    w = synth.baseline_rows(ty, rows, cols, rng)
    x = rng.standard_normal((ntok, cols)).astype(np.float32)
    got = gpu_qmv(torch, lib, ty, w, rows, cols, x, ntok, fast=fast)
    ref = oracle_mod.qmv(int(ty), w, rows, cols, x, ntok)
    for t in range(ntok):
        assert rel_l2(got[t], ref[t]) <= REL_L2_TOL, (ty.name, ntok, t)


@pytest.mark.parametrize(
    "ty,rows,cols",
    [(T.Q4_K, 5120, 17408), (T.Q3_K, 5120, 17408), (T.Q6_K, 5120, 17408), (T.IQ4_XS, 5120, 17408),
     (T.IQ3_S, 5120, 17408), (T.IQ2_XXS, 5120, 17408), (T.Q3_K, 17408, 5120), (T.Q5_K, 10240, 5120),
     (T.Q8_0, 48, 5120), (T.Q4_K, 4096, 4096), (T.Q6_K, 5120, 6144), (T.Q6_K, 1024, 5120)],
    ids=lambda v: v.name if isinstance(v, T) else str(v))
def test_qmv_baseline_shapes(env, oracle_mod, ty, rows, cols):
    torch, lib = env
    rng = np.random.default_rng(rows + cols + int(ty))
    w = synth.baseline_rows(ty, rows, cols, rng)
    for ntok in (1, 8):
        x = rng.standard_normal((ntok, cols)).astype(np.float32)
        got = gpu_qmv(torch, lib, ty, w, rows, cols, x, ntok)
        ref = oracle_mod.qmv(int(ty), w, rows, cols, x, ntok, threads=16)
        assert rel_l2(got, ref) <= REL_L2_TOL, (ty.name, ntok)


@pytest.mark.parametrize("cols", [24576, 49152])
@pytest.mark.parametrize("ty", [T.Q6_K, T.Q3_K, T.IQ2_S, T.Q8_0], ids=lambda v: v.name)
def test_qmv_wide_inputs(env, oracle_mod, ty, cols):
    """The widest in-kernel-quantized input (24576) and a packed one (49152): activation images that push
    the workgroup to fewer waves (its LDS then holds fewer stage buffers)."""
    torch, lib = env
    rng = np.random.default_rng(cols + int(ty))
    rows = 37
    w = synth.baseline_rows(ty, rows, cols, rng)
    for ntok in (1, 3):
        x = rng.standard_normal((ntok, cols)).astype(np.float32)
        got = gpu_qmv(torch, lib, ty, w, rows, cols, x, ntok)
        ref = oracle_mod.qmv(int(ty), w, rows, cols, x, ntok)
        assert rel_l2(got, ref) <= REL_L2_TOL, (ty.name, cols, ntok)


def test_argmax_rows_semantics(env, oracle_mod):
    torch, lib = env
    rng = np.random.default_rng(3)
    n, ntok = 248320, 4
    x = rng.standard_normal((ntok, n)).astype(np.float32)
    x[1, 1000] = x[1, 5] = 50.0  # tie -> lowest index
    x[2, :] = np.nan
    x[2, 777] = 1.0  # NaN never wins
    x[3, :] = -np.inf  # no value beats -inf -> INT32_MAX like the reference kernel
    out = torch.empty(ntok, dtype=torch.int32, device="cuda")
    xd_ = dev(torch, x)
    assert lib.vq_argmax_rows(P(xd_), n, ntok, P(out), None) == 0
    torch.cuda.synchronize()
    got = out.cpu().tolist()
    assert got == oracle_mod.argmax_rows(x, n, ntok)
    assert got[1] == 5 and got[2] == 777 and got[3] == 2**31 - 1


def test_zero_and_extreme_activations(env, oracle_mod):
    torch, lib = env
    rows, cols = 16, 1024
    w = synth.baseline_rows(T.Q4_K, rows, cols, 9)
    x = np.zeros((2, cols), np.float32)
    x[1, ::7] = 3.0e4
    got = gpu_qmv(torch, lib, T.Q4_K, w, rows, cols, x, 2)
    ref = oracle_mod.qmv(int(T.Q4_K), w, rows, cols, x, 2)
    assert np.array_equal(got[0], ref[0]) and np.all(got[0] == 0)
    assert rel_l2(got[1], ref[1]) <= REL_L2_TOL


# Tokens of very different magnitudes: ordinary, tiny (down to where the CPU path's 1/d is still finite), zero and
# huge. The f16 paths give each token a power-of-two scale 2^(15 - E); below ~1e-32 that scale used to overflow.
EXTREME_TOKEN_SCALES = [1.0, 1e-35, 1e-33, 3e-31, 0.0, 1e30, 1e-3]


@pytest.mark.parametrize("route", ["prefill", "small_batch", "stream"])
@pytest.mark.parametrize("ty", [T.Q4_K, T.Q6_K, T.IQ4_XS, T.Q8_0, T.Q2_K], ids=lambda t: t.name)
def test_extreme_token_scales(env, oracle_mod, route, ty):
    """Every token within the fp32 bar of the CPU path (the zero token exactly zero) on the prefill contraction and
    the small-batch matvec (f16 MFMA; int8 MFMA for Q8_0, Q2_K and, for prefill, IQ4_XS) and on the streaming
    matvec."""
    torch, lib = env
    rows, cols = 300, 2048
    n = len(EXTREME_TOKEN_SCALES)
    rng = np.random.default_rng(4242 + int(ty))
    w = synth.baseline_rows(ty, rows, cols, rng)
    x = (rng.standard_normal((n, cols)) * np.array(EXTREME_TOKEN_SCALES)[:, None]).astype(np.float32)
    if route == "prefill":
        y = torch.full((n, rows), np.nan, dtype=torch.float32, device="cuda")
        _qgemm_ws(torch, lib, ty, wdev(torch, w), rows, cols, _pack(torch, lib, x, n, cols), n, y)
        torch.cuda.synchronize()
        got = y.cpu().numpy()
    else:
        fast = route == "small_batch"
        if fast:
            want = 1 if ty in (T.Q8_0, T.Q2_K) else 2  # VQ_PATH_MFMA_I8 / VQ_PATH_MFMA_F16
            assert lib.vq_qmv_path(int(ty), rows, cols, n, lib.vq_qmv_workspace_bytes_for(int(ty), rows, cols, n)) == want
        else:
            assert lib.vq_qmv_path(int(ty), rows, cols, n, lib.vq_qmv_workspace_bytes(cols, n)) == 0
        got = gpu_qmv(torch, lib, ty, w, rows, cols, x, n, fast=fast)
    ref = oracle_mod.qmv(int(ty), w, rows, cols, x, n)
    assert np.isfinite(got).all(), route
    for t, scale in enumerate(EXTREME_TOKEN_SCALES):
        if scale == 0.0:
            assert np.all(got[t] == 0.0)
        else:
            assert rel_l2(got[t], ref[t]) <= REL_L2_TOL, (route, ty.name, scale)


@pytest.mark.parametrize("mix", [[T.Q5_K, T.Q5_K, T.Q8_0, T.Q8_0], [T.Q8_0, T.Q6_K], [T.Q4_K, T.Q8_0, T.Q4_K],
                                 [T.IQ4_XS, T.Q8_0], [T.Q5_K, T.Q6_K, T.Q8_0], [T.Q5_K, T.Q6_K, T.Q6_K],
                                 [T.Q6_K, T.Q5_K]],
                         ids=lambda m: "+".join(t.name for t in m))
@pytest.mark.parametrize("ntok", [1, 3, 6])
def test_qmv_group_mixed_matches_oracle(env, oracle_mod, mix, ntok):
    """A grouped launch over a main type and Q8_0 (a gated-delta layer's qkv/gate + beta/alpha) == each matrix
    on its own; more than 4 tokens run as several launches; Q5_K with Q6_K (a full-attention layer's q, k, v) is
    one launch, and other mixes of two non-Q8_0 types run as one launch per type."""
    torch, lib = env
    cols = 5120
    rng = np.random.default_rng(ntok + len(mix))
    rows_list = [[640, 384, 48, 48][k % 4] for k in range(len(mix))]
    ws = [synth.baseline_rows(ty, r, cols, rng) for ty, r in zip(mix, rows_list)]
    x = rng.standard_normal((ntok, cols)).astype(np.float32)
    xd_ = dev(torch, x)
    wd = [wdev(torch, w) for w in ws]
    ys = [torch.full((ntok, r), np.nan, dtype=torch.float32, device="cuda") for r in rows_list]
    n = len(mix)
    ta = (ctypes.c_int * n)(*[int(t) for t in mix])
    wa = (ctypes.c_void_p * n)(*[P(t) for t in wd])
    ra = (ctypes.c_int * n)(*rows_list)
    ya = (ctypes.c_void_p * n)(*[P(t) for t in ys])
    assert lib.vq_qmv_group_mixed_f32(n, ta, wa, ra, ya, cols, P(xd_), ntok, None) == 0
    torch.cuda.synchronize()
    for ty, w, r, yt in zip(mix, ws, rows_list, ys):
        ref = oracle_mod.qmv(int(ty), w, r, cols, x, ntok)
        assert rel_l2(yt.cpu().numpy(), ref) <= REL_L2_TOL, (ty.name, r)


def _pack(torch, lib, x: np.ndarray, ntok: int, cols: int):
    xd_ = dev(torch, x.astype(np.float32).reshape(ntok, cols))
    xp = torch.empty(lib.vq_xpack_bytes(cols, ntok), dtype=torch.uint8, device="cuda")
    assert lib.vq_pack_x(P(xd_), ntok, cols, P(xp), None) == 0
    return xp


@pytest.mark.parametrize("ty,rows_list,cols", [(T.Q3_K, [37, 64], 2048), (T.Q8_0, [48, 48, 5], 5120),
                                               (T.Q5_K, [300, 77, 9, 128], 5120), (T.IQ2_XXS, [130, 3], 1024)],
                         ids=lambda v: v.name if isinstance(v, T) else str(v))
@pytest.mark.parametrize("ntok", [1, 3, 9])
@pytest.mark.parametrize("f32", [False, True], ids=["packed", "f32"])
def test_qmv_group_matches_oracle(env, oracle_mod, ty, rows_list, cols, ntok, f32):
    """One grouped launch over matrices sharing the activations (packed, or fp32 quantized in-kernel) ==
    each matrix on its own."""
    torch, lib = env
    rng = np.random.default_rng(sum(rows_list) + ntok)
    ws = [synth.baseline_rows(ty, r, cols, rng) for r in rows_list]
    x = rng.standard_normal((ntok, cols)).astype(np.float32)
    xp = dev(torch, x) if f32 else _pack(torch, lib, x, ntok, cols)
    wd = [wdev(torch, w) for w in ws]
    ys = [torch.full((ntok, r), np.nan, dtype=torch.float32, device="cuda") for r in rows_list]
    n = len(rows_list)
    wa = (ctypes.c_void_p * n)(*[P(t) for t in wd])
    ra = (ctypes.c_int * n)(*rows_list)
    ya = (ctypes.c_void_p * n)(*[P(t) for t in ys])
    fn = lib.vq_qmv_group_f32 if f32 else lib.vq_qmv_group
    assert fn(int(ty), n, wa, ra, ya, cols, P(xp), ntok, None) == 0
    torch.cuda.synchronize()
    for w, r, y in zip(ws, rows_list, ys):
        ref = oracle_mod.qmv(int(ty), w, r, cols, x, ntok)
        got = y.cpu().numpy()
        for t in range(ntok):
            assert rel_l2(got[t], ref[t]) <= REL_L2_TOL, (ty.name, r, t)


def _lmhead(torch, lib, ty, wd, rows, cols, x, ntok, with_logits=True):
    xd_ = dev(torch, x.astype(np.float32).reshape(ntok, cols))
    nws = lib.vq_lmhead_argmax_workspace_bytes(int(ty), rows, cols, ntok)
    assert nws > 0
    ws = torch.empty(nws, dtype=torch.uint8, device="cuda")
    out = torch.full((ntok,), -7, dtype=torch.int32, device="cuda")
    logits = torch.empty(ntok, rows, dtype=torch.float32, device="cuda") if with_logits else None
    st = lib.vq_lmhead_argmax(int(ty), P(wd), rows, cols, P(xd_), ntok, P(out), P(logits) if with_logits else None,
                              P(ws), nws, None)
    assert st == 0, lib.vq_status_string(st)
    torch.cuda.synchronize()
    return out.cpu().tolist(), (logits.cpu().numpy() if with_logits else None)


@pytest.mark.parametrize("ty,rows,cols", [(T.Q6_K, 4099, 1024), (T.Q8_0, 2000, 512), (T.Q4_K, 777, 9216)],
                         ids=lambda v: v.name if isinstance(v, T) else str(v))
@pytest.mark.parametrize("ntok", [1, 3, 9])
def test_lmhead_argmax_fused(env, oracle_mod, ty, rows, cols, ntok):
    """Fused LM-head argmax: the index of the largest logit (exactly that of the logits it also writes),
    ties to the lowest row, NaN rows never win; agrees with the reference CPU logits."""
    torch, lib = env
    rng = np.random.default_rng(rows + ntok)
    w = synth.baseline_rows(ty, rows, cols, rng)
    x = rng.standard_normal((ntok, cols)).astype(np.float32)
    ref = oracle_mod.qmv(int(ty), w, rows, cols, x, ntok)
    rb = len(w) // rows
    # Tie: copy token 0's best row over a lower row; NaN: a row whose fp16 scale is NaN.
    best0 = int(np.argmax(ref[0]))
    low = best0 // 2
    w = w.copy()
    w[low * rb:(low + 1) * rb] = w[best0 * rb:(best0 + 1) * rb]
    nan_row = (best0 + 1) % rows if (best0 + 1) % rows != low else (best0 + 2) % rows
    d_off = {T.Q6_K: 208, T.Q8_0: 0, T.Q4_K: 0}[ty]
    w[nan_row * rb + d_off: nan_row * rb + d_off + 2] = np.frombuffer(np.float16(np.nan).tobytes(), np.uint8)
    ref = oracle_mod.qmv(int(ty), w, rows, cols, x, ntok)
    wd = wdev(torch, w)
    idx, logits = _lmhead(torch, lib, ty, wd, rows, cols, x, ntok)
    idx2, _ = _lmhead(torch, lib, ty, wd, rows, cols, x, ntok, with_logits=False)
    assert idx == idx2
    assert idx == oracle_mod.argmax_rows(logits, rows, ntok)  # exactly the argmax of its own logits
    assert idx[0] == low  # the tie goes to the lower row
    for t in range(ntok):
        assert np.isnan(logits[t, nan_row]) and idx[t] != nan_row
        finite = np.where(np.isnan(ref[t]), -np.inf, ref[t])
        assert finite[idx[t]] >= finite.max() - 1e-4 * np.abs(finite).max(), t
        assert rel_l2(np.nan_to_num(logits[t]), np.nan_to_num(ref[t])) <= REL_L2_TOL


@pytest.mark.parametrize("ty", QUANT_TYPES, ids=lambda t: t.name)
@pytest.mark.parametrize("rows,cols,M", [(130, 1024, 17), (64, 512, 200)])
def test_qgemm_matches_oracle(env, oracle_mod, ty, rows, cols, M):
    """The MFMA prefill contraction on the same int8 activations: within the fp32 bar of the CPU path,
    for ragged row and token tiles."""
    torch, lib = env
    rng = np.random.default_rng(rows * M + int(ty))
    w = synth.baseline_rows(ty, rows, cols, rng)
    x = rng.standard_normal((M, cols)).astype(np.float32)
    xp = _pack(torch, lib, x, M, cols)
    y = torch.full((M, rows), np.nan, dtype=torch.float32, device="cuda")
    wd = wdev(torch, w)
    st = lib.vq_qgemm(int(ty), P(wd), rows, cols, P(xp), M, P(y), None)
    assert st == 0, lib.vq_status_string(st)
    torch.cuda.synchronize()
    got = y.cpu().numpy()
    ref = oracle_mod.qmv(int(ty), w, rows, cols, x, M, threads=16)
    assert np.isfinite(got).all()
    for t in range(M):
        assert rel_l2(got[t], ref[t]) <= REL_L2_TOL, (ty.name, t)


def _qgemm_ws(torch, lib, ty, w_dev, rows, cols, xp, M, y):
    need = lib.vq_qgemm_workspace_bytes(int(ty), rows, cols, M)
    ws = torch.empty(max(need, 16), dtype=torch.uint8, device="cuda")
    st = lib.vq_qgemm_ws(int(ty), P(w_dev), rows, cols, P(xp), M, P(y), P(ws), need, None)
    assert st == 0, lib.vq_status_string(st)
    return need


@pytest.mark.parametrize("ty", [T.Q4_K, T.Q5_K, T.Q3_K, T.Q6_K, T.Q2_K, T.IQ2_XS, T.IQ2_XXS, T.IQ2_S, T.IQ3_XXS],
                         ids=lambda t: t.name)
@pytest.mark.parametrize("rows,cols,M", [(300, 2048, 50), (256, 256, 130), (520, 1024, 129), (17, 512, 1),
                                         (64, 2560, 300)])
def test_qgemm_f16_matches_oracle(env, oracle_mod, ty, rows, cols, M):
    """The f16-MFMA prefill contraction (exact code * scale, activations as two f16): within the fp32 bar of
    the CPU path for ragged row/token tiles, one or several K splits, and bit-identical on a second run."""
    torch, lib = env
    rng = np.random.default_rng(rows * 7 + M + int(ty))
    w = synth.baseline_rows(ty, rows, cols, rng)
    x = rng.standard_normal((M, cols)).astype(np.float32)
    x[:, :32] *= 1e-3  # a group far below the token's maximum
    xp = _pack(torch, lib, x, M, cols)
    wd = wdev(torch, w)
    y = torch.full((M, rows), np.nan, dtype=torch.float32, device="cuda")
    assert _qgemm_ws(torch, lib, ty, wd, rows, cols, xp, M, y) > 0
    torch.cuda.synchronize()
    got = y.cpu().numpy()
    ref = oracle_mod.qmv(int(ty), w, rows, cols, x, M, threads=16)
    assert np.isfinite(got).all()
    for t in range(M):
        assert rel_l2(got[t], ref[t]) <= REL_L2_TOL, (ty.name, t)
    y2 = torch.full((M, rows), np.nan, dtype=torch.float32, device="cuda")
    _qgemm_ws(torch, lib, ty, wd, rows, cols, xp, M, y2)
    torch.cuda.synchronize()
    assert np.array_equal(y2.cpu().numpy(), got)


@pytest.mark.parametrize("ty,rows,cols", [(T.Q4_K, 17408, 5120), (T.Q4_K, 5120, 17408), (T.Q5_K, 4096, 5120),
                                          (T.Q3_K, 17408, 5120), (T.Q6_K, 5120, 17408), (T.Q2_K, 17408, 5120),
                                          (T.IQ2_XS, 5120, 17408), (T.IQ2_XXS, 17408, 5120), (T.IQ2_S, 5120, 17408),
                                          (T.IQ3_XXS, 17408, 5120)],
                         ids=lambda v: v.name if isinstance(v, T) else str(v))
def test_qgemm_f16_prefill_shapes(env, oracle_mod, ty, rows, cols):
    """The benchmark's prefill shapes at 512 tokens (several K splits on the narrow one), all 512 tokens compared."""
    torch, lib = env
    M = 512
    rng = np.random.default_rng(rows + cols + 1)
    w = synth.baseline_rows(ty, rows, cols, rng)
    x = rng.standard_normal((M, cols)).astype(np.float32)
    xp = _pack(torch, lib, x, M, cols)
    y = torch.empty(M, rows, dtype=torch.float32, device="cuda")
    _qgemm_ws(torch, lib, ty, wdev(torch, w), rows, cols, xp, M, y)
    torch.cuda.synchronize()
    got = y.cpu().numpy()
    ref = oracle_mod.qmv(int(ty), w, rows, cols, x, M, threads=16)
    for t in range(M):  # every token: each 128-token tile and every stream-K share of the K range
        assert rel_l2(got[t], ref[t]) <= REL_L2_TOL, (ty.name, t)


@pytest.mark.parametrize("ty", [T.Q8_0, T.IQ3_S, T.IQ4_XS], ids=lambda t: t.name)
def test_qgemm_ws_other_types_run_the_int8_path(env, oracle_mod, ty):
    torch, lib = env
    rows, cols, M = 70, 512, 20
    rng = np.random.default_rng(5)
    w = synth.baseline_rows(ty, rows, cols, rng)
    x = rng.standard_normal((M, cols)).astype(np.float32)
    xp = _pack(torch, lib, x, M, cols)
    y = torch.empty(M, rows, dtype=torch.float32, device="cuda")
    assert lib.vq_qgemm_workspace_bytes(int(ty), rows, cols, M) == 0
    assert lib.vq_qgemm_ws(int(ty), P(wdev(torch, w)), rows, cols, P(xp), M, P(y), None, 0, None) == 0
    torch.cuda.synchronize()
    ref = oracle_mod.qmv(int(ty), w, rows, cols, x, M)
    assert rel_l2(y.cpu().numpy(), ref) <= REL_L2_TOL


@pytest.mark.parametrize("ty,rows,cols", [(T.Q4_K, 17408, 5120), (T.Q4_K, 5120, 17408), (T.Q3_K, 1000, 5120)],
                         ids=lambda v: v.name if isinstance(v, T) else str(v))
def test_qgemm_prefill_shapes(env, oracle_mod, ty, rows, cols):
    torch, lib = env
    M = 512
    rng = np.random.default_rng(rows + cols)
    w = synth.baseline_rows(ty, rows, cols, rng)
    x = rng.standard_normal((M, cols)).astype(np.float32)
    xp = _pack(torch, lib, x, M, cols)
    y = torch.empty(M, rows, dtype=torch.float32, device="cuda")
    assert lib.vq_qgemm(int(ty), P(wdev(torch, w)), rows, cols, P(xp), M, P(y), None) == 0
    torch.cuda.synchronize()
    got = y.cpu().numpy()
    ref = oracle_mod.qmv(int(ty), w, rows, cols, x, M, threads=16)
    for t in range(M):
        assert rel_l2(got[t], ref[t]) <= REL_L2_TOL, (ty.name, t)


@pytest.mark.parametrize("ty", ALL_TYPES, ids=lambda t: t.name)
@pytest.mark.parametrize("ntok", [6, 8, 11, 16])
def test_qmv_mfma_small_batch_matches_oracle(env, oracle_mod, ty, ntok):
    """The int8-MFMA small-batch matvec (6..16 tokens) on ragged 16-row blocks."""
    torch, lib = env
    rows, cols = 37, 2048 if ty not in (T.F32, T.F16) else 1024
    rng = np.random.default_rng(7000 + 100 * ntok + int(ty))
    w = synth.baseline_rows(ty, rows, cols, rng)
    x = rng.standard_normal((ntok, cols)).astype(np.float32)
    got = gpu_qmv(torch, lib, ty, w, rows, cols, x, ntok, fast=True)
    ref = oracle_mod.qmv(int(ty), w, rows, cols, x, ntok)
    for t in range(ntok):
        assert rel_l2(got[t], ref[t]) <= REL_L2_TOL, (ty.name, ntok, t)


@pytest.mark.parametrize("ty", [T.Q3_K, T.Q4_K, T.Q5_K, T.Q6_K, T.IQ2_XXS, T.IQ2_XS, T.IQ2_S, T.IQ3_XXS, T.IQ3_S,
                                T.IQ4_XS], ids=lambda t: t.name)
@pytest.mark.parametrize("ntok,rows,cols", [(5, 300, 768), (6, 17, 256), (7, 513, 2048), (8, 256, 1280),
                                            (16, 40, 768), (3, 40, 17408), (4, 33, 17408)])
def test_qmv_small16_matches_oracle(env, oracle_mod, ty, ntok, rows, cols):
    """The f16-MFMA small-batch matvec (5..16 tokens; 3..4 where the streaming kernel would need two passes), for
    the K-quants and the IQ types (signed codes; IQ3_S and IQ4_XS as two exact f16 terms): ragged row blocks, a
    short last K range, one K range without partials, tokens of very different magnitudes (per-token scales),
    bit-identical on a rerun."""
    torch, lib = env
    assert lib.vq_qmv_path(int(ty), rows, cols, ntok, lib.vq_qmv_workspace_bytes_for(int(ty), rows, cols, ntok)) == 2
    rng = np.random.default_rng(9000 + 37 * ntok + rows + int(ty))
    w = synth.baseline_rows(ty, rows, cols, rng)
    x = rng.standard_normal((ntok, cols)).astype(np.float32)
    x[0] *= 1e-3
    x[-1, :64] *= 40.0
    got = gpu_qmv(torch, lib, ty, w, rows, cols, x, ntok, fast=True)
    ref = oracle_mod.qmv(int(ty), w, rows, cols, x, ntok)
    for t in range(ntok):
        assert rel_l2(got[t], ref[t]) <= REL_L2_TOL, (ty.name, ntok, t)
    assert np.array_equal(gpu_qmv(torch, lib, ty, w, rows, cols, x, ntok, fast=True), got)


@pytest.mark.parametrize("ty,rows,cols", [(T.Q3_K, 17408, 5120), (T.Q4_K, 5120, 17408), (T.Q6_K, 5120, 6144),
                                          (T.IQ2_XXS, 5120, 17408), (T.IQ4_XS, 5120, 17408), (T.IQ3_S, 5120, 17408),
                                          (T.Q8_0, 48, 5120), (T.Q2_K, 1000, 5120), (T.Q5_K, 1000, 5120)],
                         ids=lambda v: v.name if isinstance(v, T) else str(v))
def test_qmv_mfma_baseline_shapes(env, oracle_mod, ty, rows, cols):
    """Split-K (several K ranges summed by the second kernel) at the sweep's shapes, batch 8 and 16."""
    torch, lib = env
    rng = np.random.default_rng(rows * 7 + cols + int(ty))
    w = synth.baseline_rows(ty, rows, cols, rng)
    for ntok in (8, 16):
        x = rng.standard_normal((ntok, cols)).astype(np.float32)
        got = gpu_qmv(torch, lib, ty, w, rows, cols, x, ntok, fast=True)
        ref = oracle_mod.qmv(int(ty), w, rows, cols, x, ntok, threads=16)
        assert rel_l2(got, ref) <= REL_L2_TOL, (ty.name, ntok)


STAGE_FLAG_SETS = [8, 2, 10, 1, 3, 11]  # SILU_MUL, NORM, SILU_MUL|NORM, ADD, NORM|ADD, all three


@pytest.mark.parametrize("ty", [T.Q4_K, T.Q3_K, T.Q6_K, T.IQ4_XS, T.Q8_0], ids=lambda t: t.name)
@pytest.mark.parametrize("flags", STAGE_FLAG_SETS)
@pytest.mark.parametrize("ntok,rows,cols", [(1, 40, 768), (3, 33, 5120), (9, 20, 512)])
def test_qmv_staged_matches_float_reference_within_int8_bound(env, oracle_mod, ty, flags, ntok, rows, cols):
    """vq_qmv_staged (the megakernel's fused SILU_MUL / NORM staging and ADD, qwen_megakernel.cu:468-551) vs
    the float64 dequant matvec of the float64-staged activations, within the reference's int8-path bound
    1.05 * sum_g sum|w| * amax_g(v) / 254 + 1e-4 (1 + |ref|) (test_phase31b_megakernel.py:184-199); ntok 9
    spans two launches (per-chunk x2 offset); bit-identical on a rerun."""
    torch, lib = env
    rng = np.random.default_rng(4400 + 10 * flags + ntok + int(ty))
    w = synth.baseline_rows(ty, rows, cols, rng)
    x = (rng.standard_normal((ntok, cols)) * 2.0).astype(np.float32)
    x2 = rng.standard_normal((ntok, cols)).astype(np.float32)
    nw = rng.uniform(0.2, 1.5, cols).astype(np.float32)
    y0 = rng.standard_normal((ntok, rows)).astype(np.float32)
    eps = 1e-6
    wd, xd, x2d, nwd = wdev(torch, w), dev(torch, x), dev(torch, x2), dev(torch, nw)

    def run():
        y = dev(torch, y0.copy())
        st = lib.vq_qmv_staged(int(ty), P(wd), rows, cols, P(xd), P(x2d), P(nwd), eps, flags, ntok, P(y), None)
        assert st == 0, lib.vq_status_string(st)
        torch.cuda.synchronize()
        return y.cpu().numpy()

    got = run()
    v = oracle_mod.stage_x(x, x2, nw, eps, flags)
    wf = oracle_mod.dequant_rows(int(ty), w, rows, cols).astype(np.float64)
    for t in range(ntok):
        ref = wf @ v[t] + (y0[t].astype(np.float64) if flags & 1 else 0.0)
        amax = np.abs(v[t].reshape(-1, 32)).max(1)
        bound = (np.abs(wf).reshape(rows, -1, 32).sum(2) * amax / 254.0).sum(1)
        assert np.all(np.abs(got[t] - ref) <= 1.05 * bound + 1e-4 * (1 + np.abs(ref))), (ty.name, flags, t)
    assert np.array_equal(run(), got)


def test_qmv_staged_without_flags_equals_vq_qmv_and_rejects_bad_arguments(env):
    torch, lib = env
    rng = np.random.default_rng(4501)
    rows, cols, ntok = 70, 1024, 2
    w = synth.baseline_rows(T.Q5_K, rows, cols, rng)
    x = rng.standard_normal((ntok, cols)).astype(np.float32)
    wd, xd = wdev(torch, w), dev(torch, x)
    y = torch.empty(ntok, rows, dtype=torch.float32, device="cuda")
    assert lib.vq_qmv_staged(int(T.Q5_K), P(wd), rows, cols, P(xd), None, None, 0.0, 0, ntok, P(y), None) == 0
    torch.cuda.synchronize()
    assert np.array_equal(y.cpu().numpy(), gpu_qmv(torch, lib, T.Q5_K, w, rows, cols, x, ntok))
    bad = lambda **k: lib.vq_qmv_staged(k.get("ty", int(T.Q5_K)), P(wd), rows, k.get("cols", cols), P(xd),  # noqa: E731
                                         k.get("x2"), k.get("nw"), k.get("eps", 1e-6), k.get("flags", 0), ntok,
                                         P(y), None)
    assert bad(flags=4) == -4  # ARGMAX is vq_lmhead_argmax's job
    assert bad(flags=8) == -4  # SILU_MUL without x2
    assert bad(flags=2) == -4  # NORM without weights
    assert bad(flags=2, nw=P(xd), eps=-1.0) == -4
    assert bad(ty=int(T.F32)) == -1
    assert bad(cols=32768) == -2


@pytest.mark.parametrize("ty,cols,ntok", [(T.Q3_K, 5120, 8), (T.Q6_K, 5120, 5), (T.Q4_K, 512, 16), (T.Q5_K, 2048, 11),
                                          (T.IQ4_XS, 2048, 8), (T.Q4_K, 2048, 2), (T.Q6_K, 25600, 3)],
                         ids=lambda v: v.name if isinstance(v, T) else str(v))
def test_qmv_group_ws_matches_single_calls(env, oracle_mod, ty, cols, ntok):
    """vq_qmv_group_ws over three matrices of different heights: bit-identical to one vq_qmv per matrix with the
    same workspace size rules (5-16 tokens of Q3_K..Q6_K in one f16-MFMA launch over all row tiles, with one
    or several K ranges; IQ4_XS at 8 tokens matrix by matrix on int8 MFMA; 2 tokens streaming; a 25600-wide
    input packed once), and within the bar of the oracle."""
    torch, lib = env
    rng = np.random.default_rng(int(ty) * 100 + ntok + cols)
    rows = [300, 1000, 129]
    ws_np = [synth.baseline_rows(ty, r, cols, rng) for r in rows]
    x = rng.standard_normal((ntok, cols)).astype(np.float32)
    xd_ = dev(torch, x)
    wd = [wdev(torch, w) for w in ws_np]
    ys = [torch.full((ntok, r), np.nan, dtype=torch.float32, device="cuda") for r in rows]
    ra = (ctypes.c_int * 3)(*rows)
    nws = lib.vq_qmv_group_workspace_bytes(int(ty), 3, ra, cols, ntok)
    wsb = torch.empty(max(nws, 256), dtype=torch.uint8, device="cuda")
    st = lib.vq_qmv_group_ws(int(ty), 3, (ctypes.c_void_p * 3)(*[P(t) for t in wd]), ra,
                             (ctypes.c_void_p * 3)(*[P(t) for t in ys]), cols, P(xd_), ntok, P(wsb), nws, None)
    assert st == 0, lib.vq_status_string(st)
    torch.cuda.synchronize()
    for w, r, yt, wdt in zip(ws_np, rows, ys, wd):
        one = torch.full((ntok, r), np.nan, dtype=torch.float32, device="cuda")
        n1 = lib.vq_qmv_workspace_bytes_for(int(ty), r, cols, ntok)
        w1 = torch.empty(max(n1, 256), dtype=torch.uint8, device="cuda")
        assert lib.vq_qmv(int(ty), P(wdt), r, cols, P(xd_), ntok, P(one), P(w1), n1, None) == 0
        torch.cuda.synchronize()
        got = yt.cpu().numpy()
        assert np.array_equal(got.view(np.uint32), one.cpu().numpy().view(np.uint32)), r
        assert rel_l2(got, oracle_mod.qmv(int(ty), w, r, cols, x, ntok)) <= REL_L2_TOL, r


def test_iq3s_grid_setter_reaches_every_path(env, oracle_mod):
    """vq_set_iq3s_grid replaces the IQ3_S codebook for every kernel (the reference uploads it at Runtime init,
    qwen_runtime.cu:1272-1286), including the streaming kernel's pre-signed copy of it. With the grid's
    entries reversed (entry e <- entry 511 - e), the matvec of weights W equals the oracle's (default grid)
    on W with every grid index i replaced by 511 - i (qs bytes and qh bits complemented), at 1 and 2 tokens
    (pre-signed table), 3 tokens (register signs) and 8 tokens (f16-MFMA small-batch kernel, grid in LDS)."""
    torch, lib = env
    rng = np.random.default_rng(353)
    rows, cols = 200, 2048
    w = synth.baseline_rows(T.IQ3_S, rows, cols, rng)
    wflip = w.reshape(rows, cols // 256, 110).copy()
    wflip[:, :, 2:74] ^= 0xFF
    grid = np.frombuffer(oracle_mod.table("iq3s_grid"), np.uint8).reshape(512, 4)
    rev = np.ascontiguousarray(grid[::-1])
    buf = (ctypes.c_uint8 * 2048).from_buffer_copy(rev.tobytes())
    assert lib.vq_set_iq3s_grid(ctypes.addressof(buf)) == 0
    try:
        for ntok, fast in ((1, False), (2, False), (3, False), (8, True)):
            x = rng.standard_normal((ntok, cols)).astype(np.float32)
            got = gpu_qmv(torch, lib, T.IQ3_S, w, rows, cols, x, ntok, fast)
            ref = oracle_mod.qmv(int(T.IQ3_S), wflip.reshape(-1), rows, cols, x, ntok)
            assert rel_l2(got, ref) <= REL_L2_TOL, ntok
    finally:
        orig = (ctypes.c_uint8 * 2048).from_buffer_copy(grid.tobytes())
        assert lib.vq_set_iq3s_grid(ctypes.addressof(orig)) == 0
    x = rng.standard_normal((1, cols)).astype(np.float32)
    assert rel_l2(gpu_qmv(torch, lib, T.IQ3_S, w, rows, cols, x, 1),
                  oracle_mod.qmv(int(T.IQ3_S), w, rows, cols, x, 1)) <= REL_L2_TOL


def test_iq3s_grid_setter_large_magnitudes(env, oracle_mod):
    """A replacement IQ3_S grid of the default grid times 8 (magnitudes up to 120, the largest a signed byte code
    holds after negation): every weight scales by exactly 8, so each path's output is 8 x the oracle's on the
    default grid. At 8 tokens this drives the f16 small-batch kernel's two-term split (|code x scale| up to
    3720, beyond f16's exact integers); at 1 token the pre-signed table's negation of bytes >= 64."""
    torch, lib = env
    rng = np.random.default_rng(909)
    rows, cols = 160, 1536
    w = synth.baseline_rows(T.IQ3_S, rows, cols, rng)
    grid = np.frombuffer(oracle_mod.table("iq3s_grid"), np.uint8).reshape(512, 4)
    assert int(grid.max()) * 8 <= 127
    big = (ctypes.c_uint8 * 2048).from_buffer_copy((grid.astype(np.uint16) * 8).astype(np.uint8).tobytes())
    assert lib.vq_set_iq3s_grid(ctypes.addressof(big)) == 0
    try:
        for ntok, fast in ((1, False), (3, False), (8, True)):
            x = rng.standard_normal((ntok, cols)).astype(np.float32)
            got = gpu_qmv(torch, lib, T.IQ3_S, w, rows, cols, x, ntok, fast)
            ref = 8.0 * oracle_mod.qmv(int(T.IQ3_S), w, rows, cols, x, ntok)
            assert rel_l2(got, ref) <= REL_L2_TOL, ntok
    finally:
        orig = (ctypes.c_uint8 * 2048).from_buffer_copy(grid.tobytes())
        assert lib.vq_set_iq3s_grid(ctypes.addressof(orig)) == 0


@pytest.mark.parametrize("ty", [T.Q3_K, T.Q4_K, T.Q6_K, T.Q8_0, T.IQ2_XXS, T.IQ4_XS], ids=lambda t: t.name)
@pytest.mark.parametrize("cols,ntok", [(256, 1), (5120, 1), (6144, 1), (17408, 1), (24576, 1), (5120, 3), (17408, 2),
                                       (2048, 8), (6144, 5)])
def test_in_kernel_quantizer_equals_packed_record(env, ty, cols, ntok):
    """The streaming matvec quantizes fp32 activations itself (vq_qmv_group_f32); its outputs are bit-identical to
    the same launch over the record vq_pack_x writes (vq_qmv_group), whose quantizer is bit-exact against the
    reference CPU path (test_quantize_x_bit_exact). Includes a group of all-zero values and one of +-3e4."""
    torch, lib = env
    rng = np.random.default_rng(cols * 10 + ntok + int(ty))
    rows = [96, 40]
    ws = [synth.baseline_rows(ty, r, cols, rng) for r in rows]
    x = rng.standard_normal((ntok, cols)).astype(np.float32)
    x[0, 32:64] = 0.0
    x[-1, 96:128] = np.where(np.arange(32) % 2, 3.0e4, -3.0e4)
    wd = [wdev(torch, w) for w in ws]
    wa = (ctypes.c_void_p * 2)(*[P(t) for t in wd])
    ra = (ctypes.c_int * 2)(*rows)
    outs = []
    for f32 in (True, False):
        ys = [torch.full((ntok, r), np.nan, dtype=torch.float32, device="cuda") for r in rows]
        ya = (ctypes.c_void_p * 2)(*[P(t) for t in ys])
        xin = dev(torch, x) if f32 else _pack(torch, lib, x, ntok, cols)
        fn = lib.vq_qmv_group_f32 if f32 else lib.vq_qmv_group
        assert fn(int(ty), 2, wa, ra, ya, cols, P(xin), ntok, None) == 0
        torch.cuda.synchronize()
        outs.append([y.cpu().numpy() for y in ys])
    for a, b in zip(*outs):
        assert not np.isnan(a).any()
        assert np.array_equal(a.view(np.uint32), b.view(np.uint32))


def _staged_ws_run(torch, lib, ty, w, rows, cols, x, x2, nw, y0, eps, flags, ntok):
    nws = lib.vq_qmv_staged_workspace_bytes(int(ty), rows, cols, ntok)
    ws = torch.empty(max(nws, 256), dtype=torch.uint8, device="cuda")
    y = dev(torch, y0.copy())
    st = lib.vq_qmv_staged_ws(int(ty), P(w), rows, cols, P(x), P(x2), P(nw), eps, flags, ntok, P(y), P(ws), nws,
                              None)
    assert st == 0, lib.vq_status_string(st)
    torch.cuda.synchronize()
    return y.cpu().numpy(), nws


def _staged_bound_check(oracle_mod, ty, w, rows, cols, x, x2, nw, y0, eps, flags, got):
    """The reference's int8-path bound for staged activations (test_phase31b_megakernel.py:184-199)."""
    v = oracle_mod.stage_x(x, x2, nw, eps, flags)
    wf = oracle_mod.dequant_rows(int(ty), w, rows, cols).astype(np.float64)
    absw = np.abs(wf).reshape(rows, -1, 32).sum(2)
    for t in range(x.shape[0]):
        ref = wf @ v[t] + (y0[t].astype(np.float64) if flags & 1 else 0.0)
        amax = np.abs(v[t].reshape(-1, 32)).max(1)
        bound = (absw * amax / 254.0).sum(1)
        assert np.all(np.abs(got[t] - ref) <= 1.05 * bound + 1e-4 * (1 + np.abs(ref))), (ty.name, flags, t)


@pytest.mark.parametrize("ty", [T.Q3_K, T.Q4_K, T.Q5_K, T.Q6_K, T.IQ4_XS, T.IQ2_XXS], ids=lambda t: t.name)
@pytest.mark.parametrize("flags", [0, 1, 2, 8, 10, 11])
@pytest.mark.parametrize("ntok,rows,cols", [(5, 300, 2048), (8, 129, 512), (16, 200, 1536)])
def test_qmv_staged_small_batch_f16(env, oracle_mod, ty, flags, ntok, rows, cols):
    """vq_qmv_staged_ws on the f16-MFMA small-batch kernel (5-16 tokens): SILU_MUL / NORM staged per K range with
    the RMS prepass, ADD in the K-range sum (or in the kernel with a single 512-column range), within the reference's
    int8-path bound of the float64 staged matvec (qwen_megakernel.cu:468-551); bit-identical on a rerun; with no
    flags bit-identical to vq_qmv with its workspace (the same kernel)."""
    torch, lib = env
    rng = np.random.default_rng(8800 + 10 * flags + ntok + int(ty))
    w = synth.baseline_rows(ty, rows, cols, rng)
    x = (rng.standard_normal((ntok, cols)) * 2.0).astype(np.float32)
    x2 = rng.standard_normal((ntok, cols)).astype(np.float32)
    nw = rng.uniform(0.2, 1.5, cols).astype(np.float32)
    y0 = rng.standard_normal((ntok, rows)).astype(np.float32)
    eps = 1e-6
    wd, xd, x2d, nwd = wdev(torch, w), dev(torch, x), dev(torch, x2), dev(torch, nw)
    got, nws = _staged_ws_run(torch, lib, ty, wd, rows, cols, xd, x2d, nwd, y0, eps, flags, ntok)
    assert nws > 0  # the f16 small-batch route
    _staged_bound_check(oracle_mod, ty, w, rows, cols, x, x2, nw, y0, eps, flags, got)
    again, _ = _staged_ws_run(torch, lib, ty, wd, rows, cols, xd, x2d, nwd, y0, eps, flags, ntok)
    assert np.array_equal(again.view(np.uint32), got.view(np.uint32))
    if flags == 0:
        plain = gpu_qmv(torch, lib, ty, w, rows, cols, x, ntok, fast=True)
        assert np.array_equal(plain.view(np.uint32), got.view(np.uint32))


@pytest.mark.parametrize("ty,rows,cols,flags", [(T.Q3_K, 17408, 5120, 2), (T.Q6_K, 5120, 17408, 9)],
                         ids=["Q3_K-gate-NORM", "Q6_K-down-SILU_MUL+ADD"])
def test_qmv_staged_small_batch_f16_mlp_shapes(env, oracle_mod, ty, rows, cols, flags):
    """The MLP block's staged projections at 8 tokens (speculative verify): RMSNorm into the Q3_K gate, SiLU * up
    into the Q6_K down with the residual ADD, on the f16 small-batch path."""
    torch, lib = env
    ntok = 8
    rng = np.random.default_rng(rows + flags)
    w = synth.baseline_rows(ty, rows, cols, rng)
    x = (rng.standard_normal((ntok, cols)) * 2.0).astype(np.float32)
    x2 = rng.standard_normal((ntok, cols)).astype(np.float32)
    nw = rng.uniform(0.2, 1.5, cols).astype(np.float32)
    y0 = rng.standard_normal((ntok, rows)).astype(np.float32)
    got, nws = _staged_ws_run(torch, lib, ty, wdev(torch, w), rows, cols, dev(torch, x), dev(torch, x2),
                              dev(torch, nw), y0, 1e-6, flags, ntok)
    assert nws > 0
    _staged_bound_check(oracle_mod, ty, w, rows, cols, x, x2, nw, y0, 1e-6, flags, got)


def test_qmv_staged_ws_falls_back_to_streaming(env):
    """Without the workspace (or for 1-4 tokens, Q8_0, ...) vq_qmv_staged_ws is vq_qmv_staged, bit for bit."""
    torch, lib = env
    rng = np.random.default_rng(91)
    for ty, ntok, rows, cols in [(T.Q4_K, 8, 64, 1024), (T.Q4_K, 2, 64, 1024), (T.Q8_0, 8, 64, 1024)]:
        w = wdev(torch, synth.baseline_rows(ty, rows, cols, rng))
        x = dev(torch, rng.standard_normal((ntok, cols)).astype(np.float32))
        x2 = dev(torch, rng.standard_normal((ntok, cols)).astype(np.float32))
        nw = dev(torch, rng.uniform(0.5, 1.5, cols).astype(np.float32))
        outs = []
        for use_ws in (False, True):
            y = torch.zeros(ntok, rows, dtype=torch.float32, device="cuda")
            if use_ws:
                st = lib.vq_qmv_staged_ws(int(ty), P(w), rows, cols, P(x), P(x2), P(nw), 1e-6, 10, ntok, P(y), None, 0,
                                          None)
            else:
                st = lib.vq_qmv_staged(int(ty), P(w), rows, cols, P(x), P(x2), P(nw), 1e-6, 10, ntok, P(y), None)
            assert st == 0, lib.vq_status_string(st)
            torch.cuda.synchronize()
            outs.append(y.cpu().numpy())
        assert np.array_equal(outs[0].view(np.uint32), outs[1].view(np.uint32)), (ty.name, ntok)


@pytest.mark.parametrize("ty", [T.Q4_K, T.Q6_K, T.Q3_K, T.IQ2_XXS, T.IQ4_XS, T.Q8_0], ids=lambda t: t.name)
@pytest.mark.parametrize("rows,cols", [(1, 256), (5, 768)])
def test_tiny_matrices_every_route(env, oracle_mod, ty, rows, cols):
    """A one-row and a five-row matrix, one or three super-blocks wide, on every route: the streaming matvec (1
    and 3 tokens), the small-batch matvec (8 and 16 tokens), the prefill contraction (2 and 20 tokens), a grouped
    launch of two such matrices and the fused LM-head argmax. With one row a token's output is a single sum, whose
    relative error under fp32 reordering grows with its cancellation (up to ~5e-5 in the CPU path itself here), so
    the bar applies to each call's whole output."""
    torch, lib = env
    rng = np.random.default_rng(rows * 1000 + cols + int(ty))
    w = synth.baseline_rows(ty, rows, cols, rng)
    wd = wdev(torch, w)
    for ntok, fast in ((1, False), (3, False), (8, True), (16, True)):
        x = rng.standard_normal((ntok, cols)).astype(np.float32)
        got = gpu_qmv(torch, lib, ty, w, rows, cols, x, ntok, fast=fast)
        ref = oracle_mod.qmv(int(ty), w, rows, cols, x, ntok)
        assert rel_l2(got, ref) <= REL_L2_TOL, ("qmv", ntok)
    for M in (2, 20):
        x = rng.standard_normal((M, cols)).astype(np.float32)
        y = torch.full((M, rows), np.nan, dtype=torch.float32, device="cuda")
        _qgemm_ws(torch, lib, ty, wd, rows, cols, _pack(torch, lib, x, M, cols), M, y)
        torch.cuda.synchronize()
        got = y.cpu().numpy()
        ref = oracle_mod.qmv(int(ty), w, rows, cols, x, M)
        assert rel_l2(got, ref) <= REL_L2_TOL, ("qgemm", M)
    x = rng.standard_normal((2, cols)).astype(np.float32)
    ys = [torch.full((2, rows), np.nan, dtype=torch.float32, device="cuda") for _ in range(2)]
    wa = (ctypes.c_void_p * 2)(P(wd), P(wd))
    ra = (ctypes.c_int * 2)(rows, rows)
    ya = (ctypes.c_void_p * 2)(*[P(t) for t in ys])
    assert lib.vq_qmv_group_f32(int(ty), 2, wa, ra, ya, cols, P(dev(torch, x)), 2, None) == 0
    torch.cuda.synchronize()
    ref = oracle_mod.qmv(int(ty), w, rows, cols, x, 2)
    for y in ys:
        assert rel_l2(y.cpu().numpy(), ref) <= REL_L2_TOL, "group"
    idx, logits = _lmhead(torch, lib, ty, wd, rows, cols, x, 2)
    assert rel_l2(logits, ref) <= REL_L2_TOL, "lmhead"
    for t in range(2):
        assert idx[t] == int(np.argmax(logits[t]))


@pytest.mark.parametrize("ty,rows,cols,M,flags", [
    (T.Q4_K, 17408, 5120, 512, 0), (T.Q4_K, 5120, 17408, 512, 0), (T.Q5_K, 10240, 5120, 512, 0),
    (T.Q4_K, 70, 512, 37, 0), (T.Q5_K, 300, 1024, 129, 1), (T.Q4_K, 1000, 5120, 1, 0), (T.Q5_K, 2048, 2048, 300, 1),
    (T.Q6_K, 5120, 17408, 512, 0), (T.Q3_K, 17408, 5120, 512, 0), (T.Q6_K, 300, 1024, 129, 1), (T.Q3_K, 70, 512, 37, 0),
    (T.Q2_K, 1000, 5120, 200, 0), (T.Q2_K, 300, 1024, 129, 1), (T.IQ2_XS, 1000, 5120, 200, 0),
    (T.IQ2_XXS, 1000, 5120, 200, 1), (T.IQ2_S, 1000, 5120, 200, 0), (T.IQ3_XXS, 1000, 5120, 200, 0),
    (T.Q4_K, 300, 20480, 37, 0), (T.Q2_K, 300, 20480, 37, 0)],  # rows past the split's register-held part
    ids=lambda v: v.name if isinstance(v, T) else str(v))
def test_qgemm_f16x_matches_oracle(env, oracle_mod, ty, rows, cols, M, flags):
    """vq_qgemm_f16x_ws against f16(x)-times-exact-weights in float64, every token; tokens 0 and 1 scaled to 1e-30
    and 1e25 (their 2^e cap and a range plain fp16 cannot hold)."""
    torch, lib = env
    rng = np.random.default_rng(rows * 7 + cols + M)
    w = synth.baseline_rows(ty, rows, cols, rng)
    x = rng.standard_normal((M, cols)).astype(np.float32)
    if M > 2:
        x[0] *= np.float32(1e-30)
        x[1] *= np.float32(1e25)
    need = lib.vq_qgemm_workspace_bytes_ex(int(ty), rows, cols, M, flags)
    assert need > 0
    ws = torch.empty(need, dtype=torch.uint8, device="cuda")
    y = torch.full((M, rows), float("nan"), dtype=torch.float32, device="cuda")
    xd = torch.from_numpy(x).cuda()
    assert lib.vq_qgemm_f16x_ws(int(ty), P(wdev(torch, w)), rows, cols, P(xd), M, P(y), P(ws), need, flags, None) == 0
    torch.cuda.synchronize()
    got = y.cpu().numpy()
    ref = oracle_mod.qgemm_f16x(int(ty), w, rows, cols, x, M)
    for t in range(M):
        assert rel_l2(got[t], ref[t]) <= REL_L2_TOL, (ty.name, t)


def test_qgemm_f16x_errors(env):
    from vinf_3080ti_amd._lib import VQ_ERR_ARG, VQ_ERR_TYPE, VQ_ERR_WORKSPACE

    torch, lib = env
    rows, cols, M = 64, 512, 8
    w = torch.zeros(rows * cols, dtype=torch.uint8, device="cuda")
    x = torch.zeros(M, cols, dtype=torch.float32, device="cuda")
    y = torch.empty(M, rows, dtype=torch.float32, device="cuda")
    need = lib.vq_qgemm_workspace_bytes_ex(int(T.Q4_K), rows, cols, M, 0)
    ws = torch.empty(need, dtype=torch.uint8, device="cuda")
    args = (P(w), rows, cols, P(x), M, P(y))
    assert lib.vq_qgemm_f16x_ws(int(T.Q8_0), *args, P(ws), need, 0, None) == VQ_ERR_TYPE
    assert lib.vq_qgemm_f16x_ws(int(T.IQ3_S), *args, P(ws), need, 0, None) == VQ_ERR_TYPE
    assert lib.vq_qgemm_f16x_ws(int(T.Q4_K), *args, P(ws), need - 256, 0, None) == VQ_ERR_WORKSPACE
    assert lib.vq_qgemm_f16x_ws(int(T.Q4_K), *args, P(ws), need, 2, None) == VQ_ERR_ARG
    assert lib.vq_qgemm_f16x_ws(int(T.Q4_K), *args, P(ws), need, 0, None) == 0
    torch.cuda.synchronize()
    assert not y.cpu().numpy().any()
