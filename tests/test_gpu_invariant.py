"""Batch invariance: with VQ_GEMM_BATCH_INVARIANT (C ABI) or Runtime.set_batch_invariant (the reference's
--batch-invariant mode, qwen_cli.py:47-49, qwen_gpu.py:738-744), a token's outputs are bit-identical whatever
batch it runs in and wherever it sits in the batch; results stay within the fp32 bar of the reference CPU path.
"""
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
    return torch, lib, _lib


def _gemm(torch, lib, _lib, ty, wd, rows, cols, x, flags):
    M = x.shape[0]
    xd = torch.from_numpy(np.ascontiguousarray(x, np.float32)).cuda()
    xp = torch.empty(lib.vq_xpack_bytes(cols, M), dtype=torch.uint8, device="cuda")
    assert lib.vq_pack_x(xd.data_ptr(), M, cols, xp.data_ptr(), None) == 0
    need = lib.vq_qgemm_workspace_bytes_ex(int(ty), rows, cols, M, flags)
    ws = torch.empty(max(need, 256), dtype=torch.uint8, device="cuda")
    y = torch.full((M, rows), np.nan, dtype=torch.float32, device="cuda")
    st = lib.vq_qgemm_ws_ex(int(ty), wd.data_ptr(), rows, cols, xp.data_ptr(), M, y.data_ptr(), ws.data_ptr(), need,
                            flags, None)
    assert st == 0, lib.vq_status_string(st)
    torch.cuda.synchronize()
    return y.cpu().numpy()


@pytest.mark.parametrize("ty,rows,cols", [(T.Q4_K, 1024, 5120), (T.Q5_K, 300, 4096), (T.Q6_K, 1000, 2048),
                                          (T.IQ4_XS, 640, 2048), (T.Q3_K, 512, 3072), (T.Q2_K, 700, 2048),
                                          (T.IQ2_S, 300, 4096), (T.IQ3_XXS, 512, 2048)],
                         ids=lambda v: v.name if isinstance(v, T) else str(v))
def test_qgemm_batch_invariant(env, oracle_mod, ty, rows, cols):
    """The same tokens alone, in a batch of 7 and at rows 131 .. of a 300-token batch (a third token tile):
    bit-identical outputs under VQ_GEMM_BATCH_INVARIANT (the f16 path of Q3_K-Q6_K splits K by the matrix only;
    the int8 path of the other types takes the whole K range per tile), all within the bar."""
    torch, lib, _lib = env
    rng = np.random.default_rng(rows + cols + int(ty))
    w = synth.baseline_rows(ty, rows, cols, rng)
    buf = np.zeros(w.size + 256, np.uint8)
    buf[: w.size] = w
    wd = torch.from_numpy(buf).cuda()
    toks = rng.standard_normal((3, cols)).astype(np.float32)
    big = rng.standard_normal((300, cols)).astype(np.float32)
    big[131:134] = toks
    small = rng.standard_normal((7, cols)).astype(np.float32)
    small[4:7] = toks
    flags = _lib.VQ_GEMM_BATCH_INVARIANT
    alone = np.stack([_gemm(torch, lib, _lib, ty, wd, rows, cols, toks[i:i + 1], flags)[0] for i in range(3)])
    in7 = _gemm(torch, lib, _lib, ty, wd, rows, cols, small, flags)[4:7]
    in300 = _gemm(torch, lib, _lib, ty, wd, rows, cols, big, flags)[131:134]
    assert np.array_equal(alone.view(np.uint32), in7.view(np.uint32))
    assert np.array_equal(alone.view(np.uint32), in300.view(np.uint32))
    ref = oracle_mod.qmv(int(ty), w, rows, cols, toks, 3, threads=16)
    assert rel_l2(alone, ref) <= REL_L2_TOL


def test_runtime_batch_invariant_mode(oracle_mod):
    """Runtime.set_batch_invariant: qmv of a token alone and inside batches of 4 and 12, qmv_group and
    lmhead_argmax agree bit for bit."""
    torch = pytest.importorskip("torch")
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    from vinf_3080ti_amd.runtime import HipWeightRuntime

    rt = HipWeightRuntime()
    rt.set_batch_invariant(True)
    rng = np.random.default_rng(5)
    rows, cols = 700, 2048
    for ty in (T.Q4_K, T.Q6_K):
        w = synth.baseline_rows(ty, rows, cols, rng)
        rt.upload_raw("w", w.tobytes(), ty, cols, rows)
        tok = rng.standard_normal(cols).astype(np.float32)
        outs = []
        for n, at in ((1, 0), (4, 2), (12, 11)):
            x = rng.standard_normal((n, cols)).astype(np.float32)
            x[at] = tok
            rt.alloc("x", n * cols)
            rt.alloc("y", n * rows)
            rt.write("x", x.tobytes())
            rt.qmv("w", "x", "y", n)
            outs.append(np.array(rt.read_floats("y"), np.float32).reshape(n, rows)[at])
        assert all(np.array_equal(o.view(np.uint32), outs[0].view(np.uint32)) for o in outs), ty.name
        assert rel_l2(outs[0], oracle_mod.qmv(int(ty), w, rows, cols, tok, 1)[0]) <= REL_L2_TOL
        rt.alloc("x", 4 * cols)
        rt.write("x", np.tile(tok, 4).tobytes())
        rt.alloc("y2", 4 * rows)
        rt.qmv_group(["w"], "x", ["y2"], 4)
        g = np.array(rt.read_floats("y2"), np.float32).reshape(4, rows)
        assert np.array_equal(g[3].view(np.uint32), outs[0].view(np.uint32))
        assert rt.lmhead_argmax("w", "x", 4) == [int(np.argmax(outs[0]))] * 4

    rt.set_batch_invariant(False)
    assert rt.gemm_min_rows == 0


@pytest.mark.parametrize("elem,hd", [(4, 128), (2, 128), (2, 256)])
def test_runtime_batch_invariant_attention(elem, hd):
    """Batch-invariant paged attention, fp32 and fp16 page pools (fp16 takes the f16 prompt kernel): one
    sequence's 3-token segment alone and beside a decode token and a 20-token prompt agrees bit for bit."""
    torch = pytest.importorskip("torch")
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    from vinf_3080ti_amd.runtime import HipWeightRuntime

    rt = HipWeightRuntime()
    rt.set_batch_invariant(True)
    rng = np.random.default_rng(50 + elem + hd)
    dt = np.float32 if elem == 4 else np.float16
    heads, kvh, page, pps, slots = 8, 2, 16, 8, 3
    pt = rng.permutation(pps * slots).astype(np.int32)
    rt.alloc("pt", pt.size)
    rt.write("pt", pt.tobytes())
    rt.set_paging("pt", page, pps, slots)
    pool = (rng.standard_normal((pps * slots, kvh, page, hd)) * 0.3).astype(dt)
    for name in ("pk", "pv"):
        rt.alloc(name, pool.size, elem)
        rt.write(name, pool.tobytes())
    q1 = rng.standard_normal((3, heads, hd)).astype(np.float32)
    rt.set_segments([(1, 40, 3)])
    rt.alloc("q", q1.size)
    rt.write("q", q1.tobytes())
    rt.alloc("o", q1.size)
    print(f"invariant attention elem {elem} hd {hd}", flush=True)
    rt.attention_seg("q", "pk", "pv", "o", heads, kvh, hd)
    alone = np.array(rt.read_floats("o"), np.float32)
    assert np.isfinite(alone).all()
    others = rng.standard_normal((1 + 20, heads, hd)).astype(np.float32)
    qa = np.concatenate([others[:1], q1, others[1:]])
    n = rt.set_segments([(0, 10, 1), (1, 40, 3), (2, 5, 20)])
    assert n == 24
    rt.alloc("q", qa.size)
    rt.write("q", qa.tobytes())
    rt.alloc("o", qa.size)
    rt.attention_seg("q", "pk", "pv", "o", heads, kvh, hd)
    beside = np.array(rt.read_floats("o"), np.float32).reshape(24, heads, hd)[1:4].reshape(-1)
    assert np.array_equal(alone.view(np.uint32), beside.view(np.uint32))
