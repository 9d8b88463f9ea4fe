"""GPU parity at the exact shapes and routes the benchmark runs, through the C ABI.

- The fused LM head at its real size (Q6_K 248320 x 5120, the qwen35 vocabulary) at 1 and 4 tokens.
- The f16-MFMA small-batch matvec at the routing the MLP block and the sweep use (workspace from
  vq_qmv_workspace_bytes_for, full rows): Q6_K 5120 x 17408 at 4 and 8 tokens, Q3_K 17408 x 5120 at 8.
- Batch dependence: the same token run alone and inside batches of 4 and 8.

Bars: fp32 outputs within rel-L2 <= 1e-5 of the reference CPU path (the oracle is bit-identical to it).
"""
from __future__ import annotations

import numpy as np
import pytest

from conftest import rel_l2
from test_gpu_parity import P, REL_L2_TOL, _lmhead, dev, gpu_qmv, wdev
from vinf_3080ti_amd import GGUFTensorType as T
from vinf_3080ti_amd import synth

pytestmark = pytest.mark.gpu

VOCAB, HIDDEN, FFN = 248320, 5120, 17408


@pytest.fixture(scope="module")
def env():
    torch = pytest.importorskip("torch")
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    from vinf_3080ti_amd import _lib

    lib = _lib.load()
    assert lib.vq_init() == 0
    return torch, lib


@pytest.fixture(scope="module")
def lm_head():
    """The LM head's weights (1.04 GB of Q6_K blocks), generated once for the module."""
    return synth.baseline_rows(T.Q6_K, VOCAB, HIDDEN, 20261202)


@pytest.mark.parametrize("ntok", [1, 4])
def test_lmhead_argmax_full_vocabulary(env, oracle_mod, lm_head, ntok):
    """vq_lmhead_argmax at the model's shape: the logits within the fp32 bar of the reference CPU path, the
    index exactly the argmax of the logits it writes, and the oracle's argmax unless the two best oracle
    logits lie closer than the fp32 error of one logit (a near-tie the bar cannot order)."""
    torch, lib = env
    rng = np.random.default_rng(300 + ntok)
    x = rng.standard_normal((ntok, HIDDEN)).astype(np.float32)
    ref = oracle_mod.qmv(int(T.Q6_K), lm_head, VOCAB, HIDDEN, x, ntok, threads=16)
    wd = wdev(torch, lm_head)
    idx, logits = _lmhead(torch, lib, T.Q6_K, wd, VOCAB, HIDDEN, x, ntok)
    idx_only, _ = _lmhead(torch, lib, T.Q6_K, wd, VOCAB, HIDDEN, x, ntok, with_logits=False)
    del wd
    assert idx == idx_only
    assert idx == oracle_mod.argmax_rows(logits, VOCAB, ntok)
    for t in range(ntok):
        assert rel_l2(logits[t], ref[t]) <= REL_L2_TOL, t
        top2 = np.sort(ref[t])[-2:]
        tol = 4 * REL_L2_TOL * np.abs(ref[t]).max()
        if top2[1] - top2[0] > tol:
            assert idx[t] == int(np.argmax(ref[t])), t
        else:
            assert ref[t][idx[t]] >= top2[1] - tol, t


@pytest.mark.parametrize("ty,rows,cols,ntok", [(T.Q6_K, HIDDEN, FFN, 4), (T.Q6_K, HIDDEN, FFN, 8),
                                               (T.Q3_K, FFN, HIDDEN, 8), (T.Q4_K, HIDDEN, FFN, 4)],
                         ids=lambda v: v.name if isinstance(v, T) else str(v))
def test_small_batch_at_bench_routing(env, oracle_mod, ty, rows, cols, ntok):
    """The matrices of the MLP block and the sweep at the batch sizes where vq_qmv routes them to the
    f16-MFMA small-batch matvec (vq_qmv_path reports it), with the workspace the benchmark passes."""
    torch, lib = env
    nws = lib.vq_qmv_workspace_bytes_for(int(ty), rows, cols, ntok)
    assert lib.vq_qmv_path(int(ty), rows, cols, ntok, nws) == 2  # VQ_PATH_MFMA_F16
    rng = np.random.default_rng(rows + 3 * ntok + int(ty))
    w = synth.baseline_rows(ty, rows, cols, rng)
    x = rng.standard_normal((ntok, cols)).astype(np.float32)
    got = gpu_qmv(torch, lib, ty, w, rows, cols, x, ntok, fast=True)
    ref = oracle_mod.qmv(int(ty), w, rows, cols, x, ntok, threads=16)
    for t in range(ntok):
        assert rel_l2(got[t], ref[t]) <= REL_L2_TOL, (ty.name, t)


@pytest.mark.parametrize("ty,rows,cols", [(T.Q3_K, FFN, HIDDEN), (T.Q6_K, HIDDEN, FFN), (T.IQ4_XS, 4096, HIDDEN),
                                          (T.Q5_K, 10240, HIDDEN)],
                         ids=lambda v: v.name if isinstance(v, T) else str(v))
def test_batch_dependence_within_bar(env, oracle_mod, ty, rows, cols):
    """A token's outputs as the only token and inside batches of 4 and 8 (routed as the benchmark routes them:
    streaming kernel alone, small-batch MFMA kernels in the batches). The kernels change with the batch, so
    the fp32 sums are not bit-identical across batch sizes: every run is held to the bar against the reference
    CPU path (which is itself batch-invariant), and the runs to twice the bar against each other."""
    torch, lib = env
    rng = np.random.default_rng(rows * 7 + int(ty))
    w = synth.baseline_rows(ty, rows, cols, rng)
    batch = rng.standard_normal((8, cols)).astype(np.float32)
    ref = oracle_mod.qmv(int(ty), w, rows, cols, batch[:1], 1, threads=16)[0]
    outs = {n: gpu_qmv(torch, lib, ty, w, rows, cols, batch[:n], n, fast=True)[0] for n in (1, 4, 8)}
    for n, y in outs.items():
        assert rel_l2(y, ref) <= REL_L2_TOL, (ty.name, n)
        assert rel_l2(y, outs[1]) <= 2 * REL_L2_TOL, (ty.name, n)
    # The streaming kernel alone, run twice, is bit-identical (no timing-dependent order).
    again = gpu_qmv(torch, lib, ty, w, rows, cols, batch[:1], 1, fast=True)[0]
    assert np.array_equal(again.view(np.uint32), outs[1].view(np.uint32))
