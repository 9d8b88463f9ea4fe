"""The benchmark times hipGraph replays of the library's calls; this checks that replays compute what eager calls do.

One graph holds every kind of launch sequence the benchmark captures: grouped and mixed streaming matvecs, the
small-batch f16 and int8 paths with their K-range sums, the no-allocation matvec, the prefill contraction (split,
GEMM, reduction of split tiles; also with f16 activations), the fused LM-head argmax and the split decode attention with its merge. It is
replayed three times; before each replay its outputs are overwritten with NaN and the same calls run eagerly on
other buffers, and every replay must reproduce the eager outputs bit for bit (the kernels are deterministic).
"""
from __future__ import annotations

import ctypes

import numpy as np
import pytest

from vinf_3080ti_amd import GGUFTensorType as T
from vinf_3080ti_amd import synth

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


def test_graph_replays_match_eager_calls(env):
    torch, lib = env
    rng = np.random.default_rng(77)

    def wdev(ty, rows, cols):
        w = synth.baseline_rows(ty, rows, cols, rng)
        buf = np.zeros(w.size + 256, np.uint8)
        buf[: w.size] = w.reshape(-1)
        return torch.from_numpy(buf).cuda()

    def fdev(shape, scale=1.0, dtype=np.float32):
        return torch.from_numpy((rng.standard_normal(shape) * scale).astype(dtype)).cuda()

    def ws(nbytes):
        return torch.empty(max(int(nbytes), 256), dtype=torch.uint8, device="cuda")

    cols = 2048
    g_w = [wdev(T.Q3_K, 300, cols), wdev(T.Q3_K, 300, cols)]
    mix_t, mix_r = [int(T.Q5_K), int(T.Q6_K), int(T.Q6_K)], [640, 96, 96]
    mix_w = [wdev(T(t), r, cols) for t, r in zip(mix_t, mix_r)]
    w6, w8, w4 = wdev(T.Q6_K, 700, cols), wdev(T.Q8_0, 300, cols), wdev(T.Q4_K, 300, cols)
    head = wdev(T.Q6_K, 4099, 1024)
    x1, x8 = fdev((1, cols)), fdev((8, cols))
    xh = fdev((2, 1024))
    M = 40
    xm = fdev((M, cols))
    xp = torch.empty(lib.vq_xpack_bytes(cols, M), dtype=torch.uint8, device="cuda")
    assert lib.vq_pack_x(P(xm), M, cols, P(xp), None) == 0
    heads, kvh, hd, seq = 24, 4, 256, 300
    q = fdev((1, heads, hd))
    kc = fdev((kvh, seq + 4, hd), 0.3, np.float16)
    vc = fdev((kvh, seq + 4, hd), 1.0, np.float16)

    ws6 = ws(lib.vq_qmv_workspace_bytes_for(int(T.Q6_K), 700, cols, 8))
    ws8 = ws(lib.vq_qmv_workspace_bytes_for(int(T.Q8_0), 300, cols, 8))
    assert lib.vq_qmv_path(int(T.Q6_K), 700, cols, 8, ws6.numel()) == 2
    assert lib.vq_qmv_path(int(T.Q8_0), 300, cols, 8, ws8.numel()) == 1
    wsg = ws(lib.vq_qgemm_workspace_bytes(int(T.Q4_K), 300, cols, M))
    wsf = ws(lib.vq_qgemm_workspace_bytes(int(T.Q4_K), 300, cols, M))
    wsh = ws(lib.vq_lmhead_argmax_workspace_bytes(int(T.Q6_K), 4099, 1024, 2))
    wsa = ws(lib.vq_attention_workspace_bytes(heads, kvh, hd, seq, 1, 0))

    def outputs():
        f = lambda *s: torch.empty(*s, dtype=torch.float32, device="cuda")
        return {"group": [f(1, 300), f(1, 300)], "mixed": [f(1, r) for r in mix_r], "small16": f(8, 700),
                "int8": f(8, 300), "noalloc": f(8, 300), "gemm": f(M, 300), "gemm_f16x": f(M, 300), "logits": f(2, 4099),
                "idx": torch.empty(2, dtype=torch.int32, device="cuda"), "attn": f(1, heads, hd)}

    def run(o, stream):
        s = stream.cuda_stream
        arr = lambda c, xs: (c * len(xs))(*xs)
        assert lib.vq_qmv_group_f32(int(T.Q3_K), 2, arr(ctypes.c_void_p, [P(w) for w in g_w]),
                                    arr(ctypes.c_int, [300, 300]), arr(ctypes.c_void_p, [P(y) for y in o["group"]]),
                                    cols, P(x1), 1, s) == 0
        assert lib.vq_qmv_group_mixed_f32(3, arr(ctypes.c_int, mix_t), arr(ctypes.c_void_p, [P(w) for w in mix_w]),
                                          arr(ctypes.c_int, mix_r), arr(ctypes.c_void_p, [P(y) for y in o["mixed"]]),
                                          cols, P(x1), 1, s) == 0
        assert lib.vq_qmv(int(T.Q6_K), P(w6), 700, cols, P(x8), 8, P(o["small16"]), P(ws6), ws6.numel(), s) == 0
        assert lib.vq_qmv(int(T.Q8_0), P(w8), 300, cols, P(x8), 8, P(o["int8"]), P(ws8), ws8.numel(), s) == 0
        assert lib.vq_qmv_noalloc(int(T.Q4_K), P(w4), 300, cols, P(x8), 8, P(o["noalloc"]), s) == 0
        assert lib.vq_qgemm_ws(int(T.Q4_K), P(w4), 300, cols, P(xp), M, P(o["gemm"]), P(wsg), wsg.numel(), s) == 0
        assert lib.vq_qgemm_f16x_ws(int(T.Q4_K), P(w4), 300, cols, P(xm), M, P(o["gemm_f16x"]), P(wsf), wsf.numel(), 0,
                                    s) == 0
        assert lib.vq_lmhead_argmax(int(T.Q6_K), P(head), 4099, 1024, P(xh), 2, P(o["idx"]), P(o["logits"]),
                                    P(wsh), wsh.numel(), s) == 0
        assert lib.vq_attention_ws(P(q), P(kc), P(vc), P(o["attn"]), 2, heads, kvh, hd, seq + 4, seq, 1, 0, 0,
                                   P(wsa), wsa.numel(), s) == 0

    def flat(o):
        out = []
        for k in sorted(o):
            for t in (o[k] if isinstance(o[k], list) else [o[k]]):
                out.append((k, t))
        return out

    eager = outputs()
    run(eager, torch.cuda.current_stream())
    torch.cuda.synchronize()
    want = [(k, t.cpu().numpy().copy()) for k, t in flat(eager)]
    assert all(np.isfinite(a).all() for k, a in want if k != "idx")

    graph_out = outputs()
    g = torch.cuda.CUDAGraph()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        with torch.cuda.graph(g, stream=side):
            run(graph_out, side)
    torch.cuda.synchronize()
    for rep in range(3):
        for _, t in flat(graph_out):
            t.fill_(-1 if t.dtype == torch.int32 else float("nan"))
        other = outputs()
        run(other, torch.cuda.current_stream())  # eager work between replays, same workspaces
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        for (k, t), (_, a) in zip(flat(graph_out), want):
            got = t.cpu().numpy()
            assert np.array_equal(got.view(np.uint32) if got.dtype == np.float32 else got,
                                  a.view(np.uint32) if a.dtype == np.float32 else a), (rep, k)
        for (k, t), (_, a) in zip(flat(other), want):
            got = t.cpu().numpy()
            assert np.array_equal(got.view(np.uint32) if got.dtype == np.float32 else got,
                                  a.view(np.uint32) if a.dtype == np.float32 else a), ("eager", rep, k)
