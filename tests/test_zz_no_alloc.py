"""The no-allocation matvec vq_qmv_noalloc (static device scratch) against vq_qmv with a workspace, through the
C ABI: two calls in a row on one GPU (the second with a smaller input, so it runs over scratch the first left
behind), each against vq_qmv on the same inputs and against the reference CPU path's bar."""
from __future__ import annotations

import numpy as np
import pytest

from conftest import rel_l2
from vinf_3080ti_amd import GGUFTensorType as T
from vinf_3080ti_amd import synth

pytestmark = pytest.mark.gpu
REL_L2_TOL = 1e-5


@pytest.fixture(scope="module")
def env():
    torch = pytest.importorskip("torch")
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    from vinf_3080ti_amd import _lib

    lib = _lib.load()
    assert lib.vq_init() == 0
    return torch, lib


def _run(torch, lib, ty, w, rows, cols, x, ntok, noalloc: bool):
    buf = np.zeros(w.size + 256, np.uint8)
    buf[: w.size] = w
    wd = torch.from_numpy(buf).cuda()
    xd = torch.from_numpy(np.ascontiguousarray(x, np.float32)).cuda()
    y = torch.full((ntok, rows), np.nan, dtype=torch.float32, device="cuda")
    if noalloc:
        st = lib.vq_qmv_noalloc(int(ty), wd.data_ptr(), rows, cols, xd.data_ptr(), ntok, y.data_ptr(), None)
    else:
        nws = lib.vq_qmv_workspace_bytes_for(int(ty), rows, cols, ntok)
        ws = torch.empty(max(nws, 1), dtype=torch.uint8, device="cuda")
        st = lib.vq_qmv(int(ty), wd.data_ptr(), rows, cols, xd.data_ptr(), ntok, y.data_ptr(), ws.data_ptr(), nws,
                        None)
    assert st == 0, lib.vq_status_string(st)
    torch.cuda.synchronize()
    return y.cpu().numpy()


# (type, rows, cols, first ntok, second ntok): the f16-MFMA small-batch path with split-K partial sums in the
# scratch (Q3_K, Q6_K), the int8-MFMA path with packed activations and partial sums (IQ4_XS), a wide input
# packed into the scratch by the streaming path (Q4_K, 32768 columns), and the streaming kernel that uses none.
CASES = [(T.Q6_K, 5120, 17408, 8, 5), (T.Q3_K, 17408, 5120, 16, 6), (T.IQ4_XS, 4096, 5120, 12, 7),
         (T.Q4_K, 300, 32768, 3, 2), (T.Q5_K, 1024, 5120, 1, 1)]


@pytest.mark.parametrize("ty,rows,cols,n1,n2", CASES, ids=lambda v: v.name if isinstance(v, T) else str(v))
def test_noalloc_matches_workspace_path(env, oracle_mod, ty, rows, cols, n1, n2):
    torch, lib = env
    rng = np.random.default_rng(rows + cols + n1)
    w = synth.baseline_rows(ty, rows, cols, rng)
    for ntok in (n1, n2):  # second call smaller: the scratch still holds the first call's values
        x = rng.standard_normal((ntok, cols)).astype(np.float32)
        got = _run(torch, lib, ty, w, rows, cols, x, ntok, True)
        want = _run(torch, lib, ty, w, rows, cols, x, ntok, False)
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), (ty.name, ntok)
        ref = oracle_mod.qmv(int(ty), w, rows, cols, x, ntok, threads=16)
        assert rel_l2(got, ref) <= REL_L2_TOL, (ty.name, ntok)


def test_noalloc_rejects_what_the_scratch_cannot_hold(env):
    """A 248320-row LM head at 8 tokens needs ~80 MB of partial sums: rejected with VQ_ERR_TOO_LARGE before any
    launch; argument errors as vq_qmv's."""
    torch, lib = env
    from vinf_3080ti_amd import _lib

    rows, cols, ntok = 248320, 5120, 8
    assert lib.vq_qmv_workspace_bytes_for(int(T.Q6_K), rows, cols, ntok) > _lib.VQ_NOALLOC_SCRATCH_BYTES
    dummy = torch.zeros(64, dtype=torch.float32, device="cuda")
    p = dummy.data_ptr()
    assert lib.vq_qmv_noalloc(int(T.Q6_K), p, rows, cols, p, ntok, p, None) == _lib.VQ_ERR_TOO_LARGE
    assert lib.vq_qmv_noalloc(int(T.Q6_K), p, rows, cols + 1, p, 1, p, None) == _lib.VQ_ERR_SHAPE
    assert lib.vq_qmv_noalloc(99, p, rows, cols, p, 1, p, None) == _lib.VQ_ERR_TYPE
    assert lib.vq_qmv_noalloc(int(T.Q6_K), None, 16, 256, p, 1, p, None) == _lib.VQ_ERR_ARG
    assert b"static scratch" in lib.vq_status_string(_lib.VQ_ERR_TOO_LARGE)
