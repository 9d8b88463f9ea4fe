"""Parity of the exact launches bench.py times, at their exact shapes, through the C ABI.

The sweep's launch list comes from bench.sweep_ops (the function the benchmark itself runs), so every distinct
launch of a 27B decode step at batch 1 and 4 is checked with the entry point, type mix, row counts and width the
timed step uses: the grouped 2 x Q3_K 17408x5120 gate+up launch (the roofline kernel), the Q5_K + Q8_0 and
Q5_K + Q6_K mixed launches, the Q6_K 5120x6144 out projections, the Q4_K 5120x17408 FFN down (streaming at 1
token, vq_qmv's f16 small-batch path at 4). The LM head (Q6_K 248320x5120, fused argmax) is checked at full size
in test_gpu_shapes.py. The MLP block's launches come from bench.mlp_routing at 1, 4 and 8 tokens. Bar: rel-L2
<= 1e-5 per matrix and per token against the oracle (bit-identical to the reference CPU path).
"""
from __future__ import annotations

import ctypes

import numpy as np
import pytest

import bench
from conftest import rel_l2
from vinf_3080ti_amd import synth

pytestmark = pytest.mark.gpu
REL_L2_TOL = 1e-5


@pytest.fixture(scope="module")
def hip():
    torch = pytest.importorskip("torch")
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    return torch, bench.Hip(torch)


def _distinct_launches(lib, ntok):
    plan = bench.sweep_plan()
    ops, nws = bench.sweep_ops(lib, plan, ntok)
    seen, out = set(), []
    for op in ops:
        if op[0] in ("pack", "head"):
            continue
        idx = [op[1]] if op[0] == "qmv" else op[1]
        key = (op[0], tuple(plan[i][1:4] for i in idx), op[2] if op[0] == "group" else None)
        if key not in seen:
            seen.add(key)
            out.append((op, [plan[i][1:4] for i in idx]))
    return out, nws


def _ids():
    from vinf_3080ti_amd import _lib

    try:
        lib = _lib.load()  # host-side routing queries only; no GPU is touched
    except Exception:  # library not built: nothing to collect
        return []
    cases = []
    for ntok in (1, 4):
        launches, _ = _distinct_launches(lib, ntok)
        for op, mats in launches:
            name = "+".join(f"{bench.TYPE_NAMES[t]}:{r}x{c}" for t, r, c in mats)
            cases.append(pytest.param(ntok, len(cases), id=f"b{ntok}-{op[0]}-{name}"))
    return cases


@pytest.mark.parametrize("ntok,case", _ids())
def test_sweep_launch_matches_oracle(hip, oracle_mod, ntok, case):
    torch, h = hip
    lib = h.lib
    launches, nws = _distinct_launches(lib, ntok)
    offset = 0 if ntok == 1 else len(_distinct_launches(lib, 1)[0])
    op, mats = launches[case - offset]
    cols = mats[0][2]
    rng = np.random.default_rng(1000 * ntok + case)
    ws_np = [synth.baseline_rows(t, r, c, rng) for t, r, c in mats]
    wd = []
    for w in ws_np:
        buf = torch.zeros(w.size + 256, dtype=torch.uint8, device="cuda")
        buf[: w.size].copy_(torch.from_numpy(w))
        wd.append(buf)
    x_np = rng.standard_normal((ntok, cols)).astype(np.float32)
    x = torch.from_numpy(x_np).cuda()
    ys = [torch.full((ntok, r), float("nan"), device="cuda") for _, r, _ in mats]
    tys, rows = [t for t, _, _ in mats], [r for _, r, _ in mats]
    print(f"sweep launch {op[0]} {mats} ntok {ntok}", flush=True)
    if op[0] == "mixed":
        h.mixed_f32(tys, wd, rows, ys, cols, x, ntok)
    elif op[0] == "group" and op[2]:
        xp = h.xpack(cols, ntok)
        h.pack(x, ntok, cols, xp)
        h.group(tys[0], wd, rows, ys, cols, xp, ntok)
    elif op[0] == "group":
        h.group_f32(tys[0], wd, rows, ys, cols, x, ntok)
    else:
        assert op[0] == "qmv" and nws > 0
        ws = torch.empty(nws, dtype=torch.uint8, device="cuda")
        st = lib.vq_qmv(tys[0], wd[0].data_ptr(), rows[0], cols, x.data_ptr(), ntok, ys[0].data_ptr(),
                        ws.data_ptr(), nws, h.s())
        assert st == 0, lib.vq_status_string(st)
    torch.cuda.synchronize()
    for (t, r, c), w, y in zip(mats, ws_np, ys):
        ref = oracle_mod.qmv(t, w, r, c, x_np, ntok, threads=16)
        got = y.cpu().numpy()
        for k in range(ntok):
            assert rel_l2(got[k], ref[k]) <= REL_L2_TOL, (bench.TYPE_NAMES[t], r, c, k)


@pytest.mark.parametrize("ntok", [1, 4, 8])
def test_mlp_block_launches_match_oracle(hip, oracle_mod, ntok):
    """The SwiGLU block as bench_mlp runs it: gate+up (2 x Q3_K 17408x5120) on vq_qmv_group_ws or the grouped
    streaming launch, down (Q6_K 5120x17408) on vq_qmv with the workspace or the streaming launch."""
    torch, h = hip
    lib = h.lib
    H, F = bench.MLP_H, bench.MLP_F
    own_gu, own_d, nws = bench.mlp_routing(lib, ntok)
    rng = np.random.default_rng(77 + ntok)
    mats = [(bench.Q3_K, F, H), (bench.Q3_K, F, H), (bench.Q6_K, H, F)]
    ws_np = [synth.baseline_rows(t, r, c, rng) for t, r, c in mats]
    wd = []
    for w in ws_np:
        buf = torch.zeros(w.size + 256, dtype=torch.uint8, device="cuda")
        buf[: w.size].copy_(torch.from_numpy(w))
        wd.append(buf)
    x_np = rng.standard_normal((ntok, H)).astype(np.float32)
    h_np = rng.standard_normal((ntok, F)).astype(np.float32)
    x, hx = torch.from_numpy(x_np).cuda(), torch.from_numpy(h_np).cuda()
    g, u, d = (torch.full((ntok, F), float("nan"), device="cuda"), torch.full((ntok, F), float("nan"), device="cuda"),
               torch.full((ntok, H), float("nan"), device="cuda"))
    ws = torch.empty(max(nws, 1), dtype=torch.uint8, device="cuda")
    print(f"mlp block ntok {ntok} own_gu {own_gu} own_d {own_d}", flush=True)
    if own_gu:
        st = lib.vq_qmv_group_ws(bench.Q3_K, 2, (ctypes.c_void_p * 2)(wd[0].data_ptr(), wd[1].data_ptr()),
                                 (ctypes.c_int * 2)(F, F), (ctypes.c_void_p * 2)(g.data_ptr(), u.data_ptr()), H,
                                 x.data_ptr(), ntok, ws.data_ptr(), nws, h.s())
        assert st == 0, lib.vq_status_string(st)
    else:
        h.group_f32(bench.Q3_K, wd[:2], [F, F], [g, u], H, x, ntok)
    if own_d:
        st = lib.vq_qmv(bench.Q6_K, wd[2].data_ptr(), H, F, hx.data_ptr(), ntok, d.data_ptr(), ws.data_ptr(), nws,
                        h.s())
        assert st == 0, lib.vq_status_string(st)
    else:
        h.group_f32(bench.Q6_K, wd[2:], [H], [d], F, hx, ntok)
    torch.cuda.synchronize()
    for (t, r, c), w, y, xin in zip(mats, ws_np, (g, u, d), (x_np, x_np, h_np)):
        ref = oracle_mod.qmv(t, w, r, c, xin, ntok, threads=16)
        got = y.cpu().numpy()
        for k in range(ntok):
            assert rel_l2(got[k], ref[k]) <= REL_L2_TOL, (bench.TYPE_NAMES[t], r, c, k)
