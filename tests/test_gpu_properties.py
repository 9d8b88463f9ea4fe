"""Size-independent properties at the benchmark's full shapes, where the CPU oracle would take minutes.

Scaling the activations by a power of two scales every output by it exactly, on every route: the CPU path's
quantizer gives the same codes (d = amax / 127 and 1 / d scale exactly), the integer partials are unchanged and
every fp32 product picks up the factor without rounding; the f16 routes' per-token 2^e moves with the token, so
their operands are the very same bits. Permuting the tokens permutes the outputs exactly (no result depends on
which other tokens share the call, for a fixed token count; for the prefill contraction only in its batch-invariant
mode). Both hold bit for bit, so they pin the routes at the
config shapes -- the grouped 2 x Q3_K 17408x5120 roofline launch, the FFN down on the streaming and small-batch
kernels, the IQ and int8 small-batch kernels, the prefill contraction at 512 tokens and the 248320-row LM head --
against themselves, complementing the oracle comparisons at smaller sizes.
"""
from __future__ import annotations

import ctypes

import numpy as np
import pytest

from vinf_3080ti_amd import GGUFTensorType as T
from vinf_3080ti_amd.synth import torch_baseline_rows

pytestmark = pytest.mark.gpu


def P(t) -> int:
    return t.data_ptr()


@pytest.fixture(scope="module")
def env():
    torch = pytest.importorskip("torch")
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    from vinf_3080ti_amd import _lib

    lib = _lib.load()
    assert lib.vq_init() == 0
    return torch, lib


def _same(a, b) -> bool:
    return np.array_equal(np.asarray(a, np.float32).view(np.uint32), np.asarray(b, np.float32).view(np.uint32))


def _check(torch, run, x, permute=True):
    """run(x) -> np.ndarray [ntok][...]; power-of-two scaling and token permutation, bit for bit."""
    y = run(x)
    assert np.isfinite(y).all()
    assert _same(run(x * 4.0), y * 4.0), "y(4x) != 4 y(x)"
    assert _same(run(x * 0.125), y * 0.125), "y(x/8) != y(x)/8"
    n = x.shape[0]
    if n > 1 and permute:
        perm = torch.from_numpy(np.random.default_rng(n).permutation(n)).cuda()
        assert _same(run(x[perm].contiguous()), y[perm.cpu().numpy()]), "token permutation"


@pytest.mark.parametrize("ty,rows,cols,ntok,ws", [
    (T.Q4_K, 5120, 17408, 1, "min"), (T.Q4_K, 5120, 17408, 4, "min"), (T.Q6_K, 5120, 17408, 8, "full"),
    (T.Q3_K, 17408, 5120, 8, "full"), (T.IQ2_XXS, 5120, 17408, 8, "full"), (T.IQ4_XS, 5120, 17408, 2, "min"),
    (T.Q8_0, 5120, 5120, 8, "full"), (T.Q5_K, 10240, 5120, 3, "min")],
    ids=lambda v: v.name if isinstance(v, T) else str(v))
def test_qmv_scaling_and_permutation(env, ty, rows, cols, ntok, ws):
    torch, lib = env
    w = torch_baseline_rows(ty, rows, cols, 17 + int(ty), "cuda")
    nws = (lib.vq_qmv_workspace_bytes_for(int(ty), rows, cols, ntok) if ws == "full"
           else lib.vq_qmv_workspace_bytes(cols, ntok))
    wk = torch.empty(max(nws, 256), dtype=torch.uint8, device="cuda")

    def run(x):
        y = torch.full((ntok, rows), float("nan"), dtype=torch.float32, device="cuda")
        assert lib.vq_qmv(int(ty), P(w), rows, cols, P(x), ntok, P(y), P(wk), nws, None) == 0
        torch.cuda.synchronize()
        return y.cpu().numpy()

    _check(torch, run, torch.randn(ntok, cols, device="cuda"))


@pytest.mark.parametrize("ntok", [1, 4])
def test_grouped_gate_up_scaling_and_permutation(env, ntok):
    """The sweep's roofline launch: 2 x Q3_K 17408x5120 in one vq_qmv_group_f32 call."""
    torch, lib = env
    rows, cols = 17408, 5120
    ws = [torch_baseline_rows(T.Q3_K, rows, cols, 3 + k, "cuda") for k in range(2)]

    def run(x):
        ys = [torch.full((ntok, rows), float("nan"), dtype=torch.float32, device="cuda") for _ in range(2)]
        assert lib.vq_qmv_group_f32(int(T.Q3_K), 2, (ctypes.c_void_p * 2)(*[P(w) for w in ws]),
                                    (ctypes.c_int * 2)(rows, rows), (ctypes.c_void_p * 2)(*[P(y) for y in ys]),
                                    cols, P(x), ntok, None) == 0
        torch.cuda.synchronize()
        return np.concatenate([y.cpu().numpy() for y in ys], axis=1)

    _check(torch, run, torch.randn(ntok, cols, device="cuda"))


@pytest.mark.parametrize("ty,rows,cols", [(T.Q4_K, 17408, 5120), (T.Q6_K, 5120, 17408), (T.Q2_K, 17408, 5120),
                                          (T.IQ2_XS, 5120, 17408), (T.IQ3_S, 5120, 5120)],
                         ids=lambda v: v.name if isinstance(v, T) else str(v))
@pytest.mark.parametrize("flags", [0, 1], ids=["stream_k", "batch_invariant"])
def test_prefill_scaling_and_permutation(env, ty, rows, cols, flags):
    """The prefill contraction at 512 tokens (f16 path for the K-quants, int8 for IQ3_S). Token permutation is
    checked in batch-invariant mode (VQ_GEMM_BATCH_INVARIANT): the default stream-K plan cuts each 128-token tile's
    K range at its own boundaries, so a token's sums may be grouped differently in another tile."""
    torch, lib = env
    M = 512
    w = torch_baseline_rows(ty, rows, cols, 29 + int(ty), "cuda")
    need = lib.vq_qgemm_workspace_bytes_ex(int(ty), rows, cols, M, flags)
    wk = torch.empty(max(need, 256), dtype=torch.uint8, device="cuda")
    xp = torch.empty(lib.vq_xpack_bytes(cols, M), dtype=torch.uint8, device="cuda")

    def run(x):
        assert lib.vq_pack_x(P(x), M, cols, P(xp), None) == 0
        y = torch.full((M, rows), float("nan"), dtype=torch.float32, device="cuda")
        assert lib.vq_qgemm_ws_ex(int(ty), P(w), rows, cols, P(xp), M, P(y), P(wk), need, flags, None) == 0
        torch.cuda.synchronize()
        return y.cpu().numpy()

    _check(torch, run, torch.randn(M, cols, device="cuda"), permute=flags == 1)


@pytest.mark.parametrize("ty,rows,cols", [(T.Q4_K, 17408, 5120), (T.Q6_K, 5120, 17408), (T.Q2_K, 17408, 5120)],
                         ids=lambda v: v.name if isinstance(v, T) else str(v))
@pytest.mark.parametrize("flags", [0, 1], ids=["stream_k", "batch_invariant"])
def test_prefill_f16x_scaling_and_permutation(env, ty, rows, cols, flags):
    """vq_qgemm_f16x_ws at 512 tokens: a power of two on a token moves its 2^e, so its f16 operands keep their bits."""
    torch, lib = env
    M = 512
    w = torch_baseline_rows(ty, rows, cols, 31 + int(ty), "cuda")
    need = lib.vq_qgemm_workspace_bytes_ex(int(ty), rows, cols, M, flags)
    wk = torch.empty(need, dtype=torch.uint8, device="cuda")

    def run(x):
        y = torch.full((M, rows), float("nan"), dtype=torch.float32, device="cuda")
        assert lib.vq_qgemm_f16x_ws(int(ty), P(w), rows, cols, P(x), M, P(y), P(wk), need, flags, None) == 0
        torch.cuda.synchronize()
        return y.cpu().numpy()

    _check(torch, run, torch.randn(M, cols, device="cuda"), permute=flags == 1)


def test_lm_head_scaling_and_permutation(env):
    """The fused LM-head argmax over the full 248320-row Q6_K head: logits scale exactly, indices do not move."""
    torch, lib = env
    rows, cols, ntok = 248320, 5120, 2
    w = torch_baseline_rows(T.Q6_K, rows, cols, 41, "cuda")
    nws = lib.vq_lmhead_argmax_workspace_bytes(int(T.Q6_K), rows, cols, ntok)
    wk = torch.empty(nws, dtype=torch.uint8, device="cuda")
    idx_seen = []

    def run(x):
        idx = torch.full((ntok,), -7, dtype=torch.int32, device="cuda")
        logits = torch.full((ntok, rows), float("nan"), dtype=torch.float32, device="cuda")
        assert lib.vq_lmhead_argmax(int(T.Q6_K), P(w), rows, cols, P(x), ntok, P(idx), P(logits), P(wk), nws,
                                    None) == 0
        torch.cuda.synchronize()
        lg = logits.cpu().numpy()
        got = idx.cpu().numpy()
        assert all(int(got[t]) == int(np.argmax(lg[t])) for t in range(ntok))
        idx_seen.append(sorted(got.tolist()))
        return lg

    _check(torch, run, torch.randn(ntok, cols, device="cuda"))
    assert all(s == idx_seen[0] for s in idx_seen)
