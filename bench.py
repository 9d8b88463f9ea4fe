"""Benchmark of the quantized-matvec hot path on one MI355X.

Headline workload: a qwen35-27B-shaped decode-step weight sweep, batch 1 — 64
layers (48 gated-delta SSM + 16 gated-attention) with a UD-Q3_K_XL-like quant mix and the Q6_K LM head with
on-device argmax, 13.44 GiB of synthetic seeded raw GGUF blocks resident in HBM. One step = one sweep:
every weight matrix of the step read once: one grouped launch per run of same-type matrices sharing an
input (<= 4; vq_qmv_group_f32, which quantizes the fp32 activations in-kernel), and the fused
vq_lmhead_argmax for the LM head.
`value` = algorithmic bytes of the step / step time (GB/s); `ms_per_step` = ms per sweep.

Also reported: per-quant-type matvec throughput at 5120x17408 (configs[0..2] shapes, rotating over weight
copies larger than the 256 MB MALL), the roofline of the dominant kernel (HIP events on its stream), and
the reference CPU path (its bit-identical C restatement) timed on this host.

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--ntok 1] [--no-graph] [--no-cpu]
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

HBM_PEAK_GBPS = 8000.0  # MI355X HBM3E, AMD-published
METRIC = "achieved HBM GB/s (% of MI355X peak) per quant type; ms per 27B decode-step sweep"

# Per-layer matrices (name, type, rows, cols, input group); shapes from qwen_tensors.py:98-118 via the
# survey's config 4. Full attention at layers 3, 7, ..., 63 (test_phase29_qwen_ops.py:207-209).
Q2_K, Q3_K, Q4_K, Q5_K, Q6_K, Q8_0, IQ4_XS, IQ3_S, IQ2_XXS, IQ2_XS, IQ2_S, IQ3_XXS = 10, 11, 12, 13, 14, 8, 23, 21, 16, 17, 22, 18
SSM_LAYER = [
    ("ssm.qkv", Q5_K, 10240, 5120, "in"),
    ("ssm.gate", Q5_K, 6144, 5120, "in"),
    ("ssm.beta", Q8_0, 48, 5120, "in"),
    ("ssm.alpha", Q8_0, 48, 5120, "in"),
    ("ssm.out", Q6_K, 5120, 6144, "out"),
]
ATTN_LAYER = [
    ("attn.q", Q5_K, 12288, 5120, "in"),
    ("attn.k", Q6_K, 1024, 5120, "in"),
    ("attn.v", Q6_K, 1024, 5120, "in"),
    ("attn.out", Q6_K, 5120, 6144, "out"),
]
FFN = [
    ("ffn.gate", Q3_K, 17408, 5120, "ffn_in"),
    ("ffn.up", Q3_K, 17408, 5120, "ffn_in"),
    ("ffn.down", Q4_K, 5120, 17408, "down"),
]
LM_HEAD = ("output", Q6_K, 248320, 5120, "head")
N_LAYERS = 64


def sweep_plan():
    """[(name, type, rows, cols, input-key)] of one decode step in execution order."""
    plan = []
    for layer in range(N_LAYERS):
        mix = ATTN_LAYER if layer % 4 == 3 else SSM_LAYER
        for name, ty, rows, cols, grp in mix + FFN:
            plan.append((f"blk.{layer}.{name}", ty, rows, cols, f"{layer}.{grp}"))
    plan.append(LM_HEAD[:4] + ("head",))
    return plan


TYPE_NAMES = {Q2_K: "Q2_K", IQ2_XS: "IQ2_XS", IQ2_S: "IQ2_S", IQ3_XXS: "IQ3_XXS", Q3_K: "Q3_K", Q4_K: "Q4_K", Q5_K: "Q5_K", Q6_K: "Q6_K", Q8_0: "Q8_0", IQ4_XS: "IQ4_XS",
              IQ3_S: "IQ3_S", IQ2_XXS: "IQ2_XXS"}
FUSED_QUANT_MAX_COLS = 24576  # narrower inputs are quantized inside the matvec (vq_qmv_group_f32)
PER_TYPE = [Q4_K, Q3_K, IQ4_XS, IQ3_S, IQ2_XXS, Q6_K]


def profiled_traffic():
    """HBM bytes per launch of the dominant kernel from the committed rocprofv3 PMC summary (FETCH_SIZE +
    WRITE_SIZE, each scaled by the same counter's reading for a plain device copy), or None."""
    f = ROOT / "profiles" / "qmv_q3k_gateup_2x17408x5120_pmc.md"
    if not f.exists():
        return None
    for line in f.read_text().splitlines():
        if line.startswith("traffic_bytes_per_launch:"):
            return int(line.split(":")[1].strip())
    return None


def profiled_trace_us():
    """Average kernel-trace duration (µs) of the dominant launch in the committed rocprofv3 summary, or None."""
    f = ROOT / "profiles" / "qmv_q3k_gateup_2x17408x5120_pmc.md"
    if not f.exists():
        return None
    for line in f.read_text().splitlines():
        if line.startswith("trace_avg_us:"):
            return float(line.split(":")[1].strip())
    return None


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def alg_bytes(ty, rows, cols, ntok):
    from vinf_3080ti_amd import row_bytes

    return rows * row_bytes(ty, cols) + 4 * ntok * (rows + cols)


class Hip:
    """Thin layer over the C ABI with torch-owned device memory."""

    def __init__(self, torch, lib_path=None):
        from vinf_3080ti_amd import _lib

        self.torch = torch
        self.lib = _lib.load(Path(lib_path) if lib_path else None)
        _lib.check(self.lib.vq_init(), "vq_init")
        self.stream = torch.cuda.current_stream()

    def s(self):
        return self.torch.cuda.current_stream().cuda_stream

    def xpack(self, cols, ntok):
        return self.torch.empty(self.lib.vq_xpack_bytes(cols, ntok), dtype=self.torch.uint8, device="cuda")

    def pack(self, x, ntok, cols, xp):
        st = self.lib.vq_pack_x(x.data_ptr(), ntok, cols, xp.data_ptr(), self.s())
        assert st == 0, st

    def qmv(self, ty, w, rows, cols, x, ntok, y):
        st = self.lib.vq_qmv(ty, w.data_ptr(), rows, cols, x.data_ptr(), ntok, y.data_ptr(), None, 0, self.s())
        assert st == 0, st

    def qmv_packed(self, ty, w, rows, cols, xp, ntok, y):
        st = self.lib.vq_qmv_packed(ty, w.data_ptr(), rows, cols, xp.data_ptr(), ntok, y.data_ptr(), self.s())
        assert st == 0, st

    def group(self, ty, ws, rows, ys, cols, xp, ntok):
        import ctypes

        n = len(ws)
        st = self.lib.vq_qmv_group(ty, n, (ctypes.c_void_p * n)(*[w.data_ptr() for w in ws]),
                                   (ctypes.c_int * n)(*rows), (ctypes.c_void_p * n)(*[y.data_ptr() for y in ys]),
                                   cols, xp.data_ptr(), ntok, self.s())
        assert st == 0, st

    def group_f32(self, ty, ws, rows, ys, cols, x, ntok):
        import ctypes

        n = len(ws)
        st = self.lib.vq_qmv_group_f32(ty, n, (ctypes.c_void_p * n)(*[w.data_ptr() for w in ws]),
                                       (ctypes.c_int * n)(*rows), (ctypes.c_void_p * n)(*[y.data_ptr() for y in ys]),
                                       cols, x.data_ptr(), ntok, self.s())
        assert st == 0, st

    def mixed_f32(self, tys, ws, rows, ys, cols, x, ntok):
        import ctypes

        n = len(ws)
        st = self.lib.vq_qmv_group_mixed_f32(n, (ctypes.c_int * n)(*tys),
                                             (ctypes.c_void_p * n)(*[w.data_ptr() for w in ws]),
                                             (ctypes.c_int * n)(*rows), (ctypes.c_void_p * n)(*[y.data_ptr() for y in ys]),
                                             cols, x.data_ptr(), ntok, self.s())
        assert st == 0, st

    def lmhead(self, ty, w, rows, cols, x, ntok, out, ws):
        st = self.lib.vq_lmhead_argmax(ty, w.data_ptr(), rows, cols, x.data_ptr(), ntok, out.data_ptr(), None,
                                       ws.data_ptr(), ws.numel(), self.s())
        assert st == 0, st

    def argmax(self, y, n, ntok, out):
        st = self.lib.vq_argmax_rows(y.data_ptr(), n, ntok, out.data_ptr(), self.s())
        assert st == 0, st


def make_weights(torch, ty, rows, cols, seed, copies=1):
    from vinf_3080ti_amd.synth import torch_baseline_rows

    return [torch_baseline_rows(ty, rows, cols, seed + 7919 * c, "cuda") for c in range(copies)]


def time_kernel_loop(torch, fn, n_iter, graph=True, reps=1):
    """Average duration (ms) of fn(i) for i < n_iter, bracketed by HIP events on the stream the launches run
    on. With graph=True the n_iter launches are captured once in a hipGraph and replayed (back-to-back
    kernels, as in a decode step, without the host's per-launch cost), the median of `reps` timed replays after
    `reps` untimed ones (the clocks settle); else launched eagerly."""
    start, stop = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    if graph:
        g = torch.cuda.CUDAGraph()
        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(side):
            with torch.cuda.graph(g, stream=side):
                for i in range(n_iter):
                    fn(i)
        torch.cuda.synchronize()
        for _ in range(reps):  # warm
            g.replay()
        torch.cuda.synchronize()
        times = []
        for _ in range(reps):
            start.record()
            g.replay()
            stop.record()
            torch.cuda.synchronize()
            times.append(start.elapsed_time(stop) / n_iter)
        del g
        return sorted(times)[len(times) // 2]
    start.record()
    for i in range(n_iter):
        fn(i)
    stop.record()
    torch.cuda.synchronize()
    return start.elapsed_time(stop) / n_iter


def bench_matvec(torch, hip, ty, rows, cols, ntok, iters=60, min_rotation_bytes=640 << 20, group=1, reps=1):
    """Per-launch µs and GB/s of the matvec kernel alone: `group` matrices of rows x cols (one
    vq_qmv_group_f32 launch, which quantizes the fp32 activations in-kernel, as in the sweep), rotating over
    weight copies larger than the MALL; launches captured in a hipGraph."""
    from vinf_3080ti_amd import row_bytes

    nbytes = rows * row_bytes(ty, cols) * group
    copies = max(2, -(-min_rotation_bytes // nbytes))
    ws = make_weights(torch, ty, rows, cols, 1234 + ty, copies * group)
    x = torch.randn(ntok, cols, device="cuda")
    xp = hip.xpack(cols, ntok)
    hip.pack(x, ntok, cols, xp)
    ys = [torch.empty(ntok, rows, device="cuda") for _ in range(group)]

    def launch(i):
        c = i % copies
        hip.group_f32(ty, ws[c * group:(c + 1) * group], [rows] * group, ys, cols, x, ntok)

    for i in range(copies):  # warm-up
        launch(i)
    ms = time_kernel_loop(torch, launch, iters, reps=reps)
    b = alg_bytes(ty, rows, cols, ntok) * group
    del ws
    torch.cuda.empty_cache()
    return {"us": ms * 1e3, "GBps": b / (ms * 1e-3) / 1e9, "bytes": b, "frac": b / (ms * 1e-3) / 1e9 / HBM_PEAK_GBPS,
            "copies": copies}


def bench_matvec_routed(torch, hip, ty, rows, cols, ntok, iters=40, min_rotation_bytes=640 << 20):
    """One vq_qmv call with the workspace vq_qmv_workspace_bytes_for asks, so the library routes the batch the way
    a caller gets it (streaming, int8-MFMA or f16-MFMA small-batch kernel; `path`): µs, GB/s and fraction of
    8 TB/s over the call's kernels, rotating over weight copies larger than the MALL in a hipGraph."""
    from vinf_3080ti_amd import row_bytes

    nbytes = rows * row_bytes(ty, cols)
    copies = max(2, -(-min_rotation_bytes // nbytes))
    ws = make_weights(torch, ty, rows, cols, 4321 + ty, copies)
    x = torch.randn(ntok, cols, device="cuda")
    y = torch.empty(ntok, rows, device="cuda")
    nws = hip.lib.vq_qmv_workspace_bytes_for(ty, rows, cols, ntok)
    wsb = torch.empty(max(nws, 256), dtype=torch.uint8, device="cuda")
    path = hip.lib.vq_qmv_path(ty, rows, cols, ntok, nws)

    def launch(i):
        st = hip.lib.vq_qmv(ty, ws[i % copies].data_ptr(), rows, cols, x.data_ptr(), ntok, y.data_ptr(),
                            wsb.data_ptr() if nws else None, nws, hip.s())
        assert st == 0, st

    for i in range(copies):
        launch(i)
    ms = time_kernel_loop(torch, launch, iters)
    b = alg_bytes(ty, rows, cols, ntok)
    del ws
    torch.cuda.empty_cache()
    return {"us": round(ms * 1e3, 3), "GBps": round(b / (ms * 1e-3) / 1e9, 1),
            "frac": round(b / (ms * 1e-3) / 1e9 / HBM_PEAK_GBPS, 4),
            "path": {0: "stream", 1: "mfma-int8", 2: "mfma-f16"}.get(path, str(path))}


def ab_matvec(torch, hips, ty, rows, cols, ntok, group=1, reps=5, iters=100, min_rotation_bytes=640 << 20):
    """The bench_matvec launch for several builds of the library (one Hip per build) on the same weights,
    interleaved rep by rep, so that box-to-box and run-to-run drift hits every build alike: per build the
    median and minimum µs per launch over `reps` graph replays of `iters` launches."""
    import statistics

    nbytes = rows * row_bytes_of(ty, cols) * group
    copies = max(2, -(-min_rotation_bytes // nbytes))
    ws = make_weights(torch, ty, rows, cols, 1234 + ty, copies * group)
    x = torch.randn(ntok, cols, device="cuda")
    ys = [torch.empty(ntok, rows, device="cuda") for _ in range(group)]
    times = [[] for _ in hips]
    for _ in range(reps):
        for k, hip in enumerate(hips):
            def launch(i, hip=hip):
                c = i % copies
                hip.group_f32(ty, ws[c * group:(c + 1) * group], [rows] * group, ys, cols, x, ntok)

            for i in range(copies):
                launch(i)
            times[k].append(time_kernel_loop(torch, launch, iters) * 1e3)
    b = alg_bytes(ty, rows, cols, ntok) * group
    del ws
    torch.cuda.empty_cache()
    return [{"med_us": round(statistics.median(t), 3), "min_us": round(min(t), 3),
             "GBps_med": round(b / (statistics.median(t) * 1e-6) / 1e9, 1)} for t in times]


MFMA_F32_PEAK_TFLOPS = 157.3  # MI355X dense fp32 MFMA, AMD-published


def bench_ops(torch, hip):
    """The sequence ops around the matvec at the qwen35-27B shapes (48 value heads x kd 128 x vd 128 gated delta
    with a 10240-channel K=4 conv; 24 query heads over 4 kv heads, hd 256 attention), each timed alone in a
    hipGraph of back-to-back launches. HBM-bound ops report bytes per call (state read + written once, inputs,
    outputs) and their fraction of 8 TB/s; the prompt attention reports useful TFLOP/s (2 * 2 * visible
    (query, key) pairs * hd * heads) against the 2.5 PFLOP/s dense f16 MFMA peak it runs on (frac_issued counts
    both MFMAs of each hi/lo split product)."""
    import ctypes

    lib, st = hip.lib, hip.s
    kh, vh, kd, vd, K = 16, 48, 128, 128, 4
    cdim = 2 * kh * kd + vh * vd
    out = {}
    for ntok in (1, 8):
        for elem in (4, 2):
            conv = torch.randn(ntok, cdim, device="cuda")
            b, a = torch.randn(ntok, vh, device="cuda"), torch.randn(ntok, vh, device="cuda")
            sa, dt = -torch.rand(vh, device="cuda") - 0.1, torch.randn(vh, device="cuda")
            S = (torch.randn(vh * kd * vd, device="cuda") * 0.1).to(torch.float32 if elem == 4 else torch.float16)
            o = torch.empty(ntok, vh, vd, device="cuda")

            def gd(i):
                r = lib.vq_gated_delta(conv.data_ptr(), b.data_ptr(), a.data_ptr(), sa.data_ptr(), dt.data_ptr(),
                                       S.data_ptr(), elem, o.data_ptr(), kh, vh, kd, vd, 1e-6, 0, ntok, None, 1, st())
                assert r == 0, r

            ms = time_kernel_loop(torch, gd, 200)
            nb = 2 * vh * kd * vd * elem + ntok * (cdim + 2 * vh + vh * vd) * 4
            out[f"gated_delta_ntok{ntok}_state{'f32' if elem == 4 else 'f16'}"] = {
                "us": round(ms * 1e3, 3), "bytes": nb, "GBps": round(nb / (ms * 1e-3) / 1e9, 1),
                "frac": round(nb / (ms * 1e-3) / 1e9 / HBM_PEAK_GBPS, 4)}
    for ntok in (1, 8):
        x = torch.randn(ntok, cdim, device="cuda")
        state = torch.randn(cdim, K, device="cuda")
        w = torch.randn(cdim, K, device="cuda")
        y = torch.empty(ntok, cdim, device="cuda")

        def cu(i):
            r = lib.vq_conv_update(x.data_ptr(), state.data_ptr(), w.data_ptr(), y.data_ptr(), cdim, K, ntok, None, 1,
                                   st())
            assert r == 0, r

        ms = time_kernel_loop(torch, cu, 200)
        nb = (3 * cdim * K + 2 * ntok * cdim) * 4
        out[f"conv_update_ntok{ntok}"] = {"us": round(ms * 1e3, 3), "bytes": nb,
                                          "GBps": round(nb / (ms * 1e-3) / 1e9, 1),
                                          "frac": round(nb / (ms * 1e-3) / 1e9 / HBM_PEAK_GBPS, 4)}
    heads, kvh, hd = 24, 4, 256
    for ntok, seq_len in ((1, 4096), (8, 4096), (512, 1)):
        max_seq = seq_len + ntok
        q = torch.randn(ntok, heads, hd, device="cuda")
        kc = (torch.randn(kvh, max_seq, hd, device="cuda") * 0.3).half()
        vc = torch.randn(kvh, max_seq, hd, device="cuda").half()
        o = torch.empty_like(q)

        nws = lib.vq_attention_workspace_bytes(heads, kvh, hd, seq_len, ntok, 0)
        wsb = torch.empty(max(nws, 1), dtype=torch.uint8, device="cuda")

        def at(i):
            r = lib.vq_attention_ws(q.data_ptr(), kc.data_ptr(), vc.data_ptr(), o.data_ptr(), 2, heads, kvh, hd,
                                    max_seq, seq_len, ntok, 0, 0, wsb.data_ptr() if nws else None, nws, st())
            assert r == 0, r

        ms = time_kernel_loop(torch, at, 50)
        pairs = sum(seq_len + t for t in range(ntok))
        rec = {"us": round(ms * 1e3, 3)}
        if ntok > 8:
            tf = 2 * 2 * pairs * hd * heads / (ms * 1e-3) / 1e12
            rec.update(kernel="attention_prompt16 (f16 MFMA on exact hi/lo splits: 2 MFMAs per product)", tflops=round(tf, 2),
                       frac=round(tf / MFMA_F16_PEAK_TFLOPS, 4), frac_issued=round(2 * tf / MFMA_F16_PEAK_TFLOPS, 4))
        else:
            nb = 2 * kvh * (seq_len + ntok - 1) * hd * 2 + 2 * ntok * heads * hd * 4
            rec.update(kernel="attention_split16 + merge (f16 MFMA, flash decoding)", bytes=nb, GBps=round(nb / (ms * 1e-3) / 1e9, 1),
                       frac=round(nb / (ms * 1e-3) / 1e9 / HBM_PEAK_GBPS, 4))
        out[f"attention_fp16kv_ntok{ntok}_ctx{seq_len + ntok - 1}"] = rec
    return out


def row_bytes_of(ty, cols):
    from vinf_3080ti_amd import row_bytes

    return row_bytes(ty, cols)


MFMA_INT8_PEAK_TOPS = 5000.0  # MI355X dense int8 MFMA, AMD-published (no sparsity)
MFMA_F16_PEAK_TFLOPS = 2500.0  # MI355X dense f16 MFMA, AMD-published (no sparsity)


def bench_gemm(torch, hip, ty, rows, cols, M, iters=20, min_rotation_bytes=640 << 20, f16x=False):
    """Prefill contraction: M tokens x (rows x cols) weights through vq_qgemm_ws (f16
    MFMA for Q2_K-Q6_K, IQ2_XXS/XS/S and IQ3_XXS: exact code*scale weights, activations as two f16 -> two MFMAs per useful multiply-add,
    three for Q6_K (its weight as an f16 rounding plus a remainder); the int8-MFMA vq_qgemm for other types), activations packed beforehand. Reports us per launch (the
    activation split, the contraction and the reduction of split tiles), useful TFLOP/s (2*M*rows*cols) and
    its fraction of the path's dense MFMA peak; `mfma_issued_util` counts the hi/lo MFMAs actually issued.
    f16x: vq_qgemm_f16x_ws instead (fp32 activations rounded to f16 in the timed pre-pass, the reference's
    tensor-core numerics: one MFMA per product)."""
    from vinf_3080ti_amd import row_bytes

    nbytes = rows * row_bytes(ty, cols)
    copies = max(2, -(-min_rotation_bytes // nbytes))
    ws = make_weights(torch, ty, rows, cols, 4321 + ty, copies)
    x = torch.randn(M, cols, device="cuda")
    xp = hip.xpack(cols, M)
    hip.pack(x, M, cols, xp)
    y = torch.empty(M, rows, device="cuda")
    need = hip.lib.vq_qgemm_workspace_bytes(ty, rows, cols, M)
    wk = torch.empty(max(need, 256), dtype=torch.uint8, device="cuda")

    def launch(i):
        if f16x:
            st = hip.lib.vq_qgemm_f16x_ws(ty, ws[i % copies].data_ptr(), rows, cols, x.data_ptr(), M, y.data_ptr(),
                                          wk.data_ptr(), need, 0, hip.s())
        else:
            st = hip.lib.vq_qgemm_ws(ty, ws[i % copies].data_ptr(), rows, cols, xp.data_ptr(), M, y.data_ptr(),
                                     wk.data_ptr() if need else None, need, hip.s())
        assert st == 0, st

    for i in range(copies):
        launch(i)
    ms = time_kernel_loop(torch, launch, iters)
    del ws
    torch.cuda.empty_cache()
    tops = 2.0 * M * rows * cols / (ms * 1e-3) / 1e12
    f16 = need > 0
    peak = MFMA_F16_PEAK_TFLOPS if f16 else MFMA_INT8_PEAK_TOPS
    out = {"us": round(ms * 1e3, 3), "path": "f16-mfma" if f16 else "int8-mfma", "tflops": round(tops, 2),
           "mfma_util": round(tops / peak, 4), "weight_GBps": round(nbytes / (ms * 1e-3) / 1e9, 1)}
    if f16x:
        out["path"] = "f16-mfma, f16 activations"
    elif f16:  # hi/lo activation MFMAs per useful product; Q6_K adds its remainder's b_hi product
        out["mfma_issued_util"] = round((3 if ty == Q6_K else 2) * tops / peak, 4)
    return out


MLP_H, MLP_F = 5120, 17408


def mlp_routing(lib, ntok, mfma=None):
    """(gate+up on vq_qmv_group_ws, down on vq_qmv, workspace bytes) for the MLP block at ntok tokens: per matrix,
    vq_qmv's own routing with the workspace (an MFMA path) or the grouped streaming launch. mfma forces one."""
    import ctypes

    H, F = MLP_H, MLP_F
    nws = max(lib.vq_qmv_group_workspace_bytes(Q3_K, 2, (ctypes.c_int * 2)(F, F), H, ntok),
              lib.vq_qmv_workspace_bytes_for(Q6_K, H, F, ntok))
    if mfma is None:
        return lib.vq_qmv_path(Q3_K, F, H, ntok, nws) > 0, lib.vq_qmv_path(Q6_K, H, F, ntok, nws) > 0, nws
    return bool(mfma), bool(mfma), nws


def bench_mlp(torch, hip, ntok, iters=20, min_rotation_bytes=640 << 20, mfma=None):
    """the qwen35 SwiGLU MLP block's three matvecs (gate/up Q3_K 17408x5120, down
    Q6_K 5120x17408) at batch ntok, weights rotating beyond the MALL. mfma=True: vq_qmv with its workspace for
    all three (the f16-MFMA small-batch matvec for these types from 5 tokens on, and from 3 over the 17408-wide
    down input); mfma=False: the streaming kernel (grouped gate/up + down, activations quantized in-kernel).
    Default: vq_qmv (down) and vq_qmv_group_ws (gate and up together) where vq_qmv_path picks an MFMA path, else
    the grouped streaming launch."""
    from vinf_3080ti_amd import row_bytes

    H, F = 5120, 17408
    per_set = 2 * F * row_bytes(Q3_K, H) + H * row_bytes(Q6_K, F)
    copies = max(2, -(-min_rotation_bytes // per_set))
    sets = [(make_weights(torch, Q3_K, F, H, 11 + 3 * c)[0], make_weights(torch, Q3_K, F, H, 12 + 3 * c)[0],
             make_weights(torch, Q6_K, H, F, 13 + 3 * c)[0]) for c in range(copies)]
    x = torch.randn(ntok, H, device="cuda")
    h = torch.randn(ntok, F, device="cuda")
    g, u, d = (torch.empty(ntok, F, device="cuda"), torch.empty(ntok, F, device="cuda"),
               torch.empty(ntok, H, device="cuda"))
    lib = hip.lib
    import ctypes

    rows2 = (ctypes.c_int * 2)(F, F)
    own_gu, own_d, nws = mlp_routing(lib, ntok, mfma)
    ws = torch.empty(max(nws, 1), dtype=torch.uint8, device="cuda")
    path = "mfma" if own_gu and own_d else "mixed" if own_gu or own_d else "stream"

    def qmv(ty, w, rows, cols, xi, yo):
        st = lib.vq_qmv(ty, w.data_ptr(), rows, cols, xi.data_ptr(), ntok, yo.data_ptr(), ws.data_ptr(), nws,
                        hip.s())
        assert st == 0, st

    def launch(i):
        wg, wu, wd = sets[i % copies]
        if own_gu:  # gate and up in one call: one MFMA launch over both matrices' row tiles
            st = lib.vq_qmv_group_ws(Q3_K, 2, (ctypes.c_void_p * 2)(wg.data_ptr(), wu.data_ptr()), rows2,
                                     (ctypes.c_void_p * 2)(g.data_ptr(), u.data_ptr()), H, x.data_ptr(), ntok,
                                     ws.data_ptr(), nws, hip.s())
            assert st == 0, st
        else:
            hip.group_f32(Q3_K, [wg, wu], [F, F], [g, u], H, x, ntok)
        if own_d:
            qmv(Q6_K, wd, H, F, h, d)
        else:
            hip.group_f32(Q6_K, [wd], [H], [d], F, h, ntok)

    for i in range(copies):
        launch(i)
    ms = time_kernel_loop(torch, launch, iters)
    b = 2 * alg_bytes(Q3_K, F, H, ntok) + alg_bytes(Q6_K, H, F, ntok)
    del sets
    torch.cuda.empty_cache()
    return {"us": round(ms * 1e3, 2), "GBps": round(b / (ms * 1e-3) / 1e9, 1),
            "frac": round(b / (ms * 1e-3) / 1e9 / HBM_PEAK_GBPS, 4), "path": path}


def sweep_ops(lib, plan, ntok):
    """The launch sequence of one sweep step, decided on the host from the plan and vq_qmv's routing queries:
    ([("pack", cols) | ("mixed", [plan index]) | ("group", [plan index], packed) | ("qmv", i) | ("head", i)],
    workspace bytes of the ("qmv", i) calls). Per distinct input one pack when it is wider than the in-kernel
    quantizer takes, then one grouped launch per run of consecutive same-type matrices (<= 4) reading it, a mixed
    launch for a main type plus Q8_0 or for Q5_K plus Q6_K; the LM head is the fused matvec + argmax."""
    ops = []
    i = 0
    while i < len(plan):
        name, ty, rows, cols, key = plan[i]
        if name == "output":
            ops.append(("head", i))
            i += 1
            continue
        packed = cols > FUSED_QUANT_MAX_COLS
        if packed:
            ops.append(("pack", cols))
        j = i
        while j < len(plan) and plan[j][4] == key:
            run = [k for k in range(j, min(j + 4, len(plan))) if plan[k][4] == key]
            tys = {plan[k][1] for k in run}
            if len(tys) > 1 and not packed and (len(tys - {Q8_0}) == 1 or tys == {Q5_K, Q6_K}):
                ops.append(("mixed", run))
                j = run[-1] + 1
                continue
            k = j
            while k < len(plan) and k - j < 4 and plan[k][4] == key and plan[k][1] == ty and plan[k][3] == cols:
                k += 1
            ops.append(("group", list(range(j, k)), packed))
            j = k
            if j < len(plan):
                ty, cols = plan[j][1], plan[j][3]
        i = j
    # Several tokens: matrices for which vq_qmv takes an MFMA path (e.g. 3..4 tokens over the 17408-wide FFN
    # down input, which the streaming kernel reads twice) leave their group for a vq_qmv call of their own.
    nws = 0
    if ntok > 1:
        routed = []
        for op in ops:
            if op[0] != "group" or op[2]:
                routed.append(op)
                continue
            keep, own = [], []
            for i in op[1]:
                _, ty_i, rows_i, cols_i, _ = plan[i]
                need = lib.vq_qmv_workspace_bytes_for(ty_i, rows_i, cols_i, ntok)
                if lib.vq_qmv_path(ty_i, rows_i, cols_i, ntok, need) > 0:
                    own.append(i)
                    nws = max(nws, need)
                else:
                    keep.append(i)
            if keep:
                routed.append(("group", keep, False))
            routed.extend(("qmv", i) for i in own)
        ops = routed
    return ops, nws


class Sweep:
    """All weights of one 27B decode step resident in HBM, plus the per-step launch sequence."""

    def __init__(self, torch, hip, ntok, weights=None):
        self.torch, self.hip, self.ntok = torch, hip, ntok
        self.plan = sweep_plan()
        self.w = weights or [make_weights(torch, ty, rows, cols, 1 + i)[0] for i, (_, ty, rows, cols, _) in enumerate(self.plan)]
        self.bytes = sum(alg_bytes(ty, r, c, ntok) for _, ty, r, c, _ in self.plan)
        self.weight_bytes = sum(w.numel() - 256 for w in self.w)
        maxc = max(p[3] for p in self.plan)
        self.x = torch.randn(ntok, maxc, device="cuda")
        self.xp = hip.xpack(maxc, ntok)
        self.ys = {}  # one output per matrix shape of a group position (outputs are not consumed)
        self.ids = torch.empty(ntok, dtype=torch.int32, device="cuda")
        self.ops, nws = sweep_ops(hip.lib, self.plan, ntok)
        for op in self.ops:
            if op[0] == "head":
                _, ty, rows, cols, _ = self.plan[op[1]]
                nh = hip.lib.vq_lmhead_argmax_workspace_bytes(ty, rows, cols, ntok)
                self.head_ws = torch.empty(nh, dtype=torch.uint8, device="cuda")
        self.qmv_ws = torch.empty(nws, dtype=torch.uint8, device="cuda") if nws else None
        for _, _, rows, _, _ in self.plan:
            self.ys.setdefault(rows, torch.empty(ntok, rows, device="cuda"))
        self.launches = sum(2 if op[0] in ("head", "qmv") else 1 for op in self.ops)  # qmv: matvec + range sums

    def step(self):
        """One decode-step sweep: every matrix read once."""
        hip, ntok = self.hip, self.ntok
        for op in self.ops:
            if op[0] == "pack":
                hip.pack(self.x, ntok, op[1], self.xp)
            elif op[0] == "mixed":
                idx = op[1]
                cols = self.plan[idx[0]][3]
                hip.mixed_f32([self.plan[i][1] for i in idx], [self.w[i] for i in idx], [self.plan[i][2] for i in idx],
                              [self.ys[self.plan[i][2]] for i in idx], cols, self.x, ntok)
            elif op[0] == "group":
                idx = op[1]
                _, ty, _, cols, _ = self.plan[idx[0]]
                rows = [self.plan[i][2] for i in idx]
                ys = [self.ys[r] for r in rows]
                if op[2]:
                    hip.group(ty, [self.w[i] for i in idx], rows, ys, cols, self.xp, ntok)
                else:
                    hip.group_f32(ty, [self.w[i] for i in idx], rows, ys, cols, self.x, ntok)
            elif op[0] == "qmv":
                _, ty, rows, cols, _ = self.plan[op[1]]
                ws = self.qmv_ws
                st = hip.lib.vq_qmv(ty, self.w[op[1]].data_ptr(), rows, cols, self.x.data_ptr(), ntok,
                                    self.ys[rows].data_ptr(), ws.data_ptr() if ws is not None else None,
                                    ws.numel() if ws is not None else 0, hip.s())
                assert st == 0, st
            else:
                _, ty, rows, cols, _ = self.plan[op[1]]
                hip.lmhead(ty, self.w[op[1]], rows, cols, self.x, ntok, self.ids, self.head_ws)


def time_sweep(torch, sw, steps, warmup, use_graph=True):
    """ms per step of a Sweep (hipGraph-captured unless use_graph is False)."""
    for _ in range(warmup):
        sw.step()
    torch.cuda.synchronize()
    graph = None
    if use_graph:
        graph = torch.cuda.CUDAGraph()
        s = torch.cuda.Stream()
        s.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(s):
            with torch.cuda.graph(graph, stream=s):
                sw.step()
        torch.cuda.synchronize()
        for _ in range(warmup):
            graph.replay()
        torch.cuda.synchronize()
    start, stop = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    start.record()
    for _ in range(steps):
        graph.replay() if graph else sw.step()
    stop.record()
    torch.cuda.synchronize()
    return start.elapsed_time(stop) / steps, graph is not None


def host_cpu() -> dict:
    """The box's CPU as lscpu reports it, and the CPUs this process may run on."""
    info = {"model": None, "sockets": None, "physical_cores": None, "cpus_in_affinity": len(os.sched_getaffinity(0))}
    try:
        import subprocess

        out = subprocess.run(["lscpu"], capture_output=True, text=True, timeout=20).stdout
        kv = dict(line.split(":", 1) for line in out.splitlines() if ":" in line)
        kv = {k.strip(): v.strip() for k, v in kv.items()}
        info["model"] = kv.get("Model name")
        sockets = int(kv.get("Socket(s)", "0") or 0)
        per = int(kv.get("Core(s) per socket", "0") or 0)
        info["sockets"] = sockets or None
        info["physical_cores"] = sockets * per or None
    except (OSError, ValueError):
        pass
    return info


CPU_SHARE = 16  # host CPUs one GPU's share of the box may keep busy


def host_ram_bytes() -> int:
    try:
        return os.sysconf("SC_PAGE_SIZE") * os.sysconf("SC_PHYS_PAGES")
    except (ValueError, OSError):
        return 0


FULL_SWEEP_MIN_RAM = 32 << 30  # the full config-4 sweep holds 13.4 GiB of weights in host memory


def fast_baseline_rows(ty, rows, cols, rng, base):
    """synth.baseline_rows' distribution at memory speed for the 13.4 GiB CPU sweep: the block bytes are a
    16 MiB random block XORed with a per-chunk constant (a bijection per byte, so each byte stays uniform and
    every matrix occupies distinct memory), then every fp16 scale field is set to fp16(|N(0, 1e-3)|)."""
    import numpy as np

    from vinf_3080ti_amd.gguf_types import F16_FIELDS, GGUFTensorType, traits

    bs, ts = traits(ty)
    nblk = rows * cols // bs
    n64 = -(-nblk * ts // 8)
    out = np.empty(n64, np.uint64)
    salt = int(rng.integers(1, 2**62))
    for k in range(0, n64, base.size):
        m = min(base.size, n64 - k)
        np.bitwise_xor(base[:m], np.uint64((salt + k * 0x9E3779B97F4A7C15) % 2**64), out=out[k : k + m])
    blocks = out.view(np.uint8)[: nblk * ts].reshape(nblk, ts)
    for off in F16_FIELDS[GGUFTensorType(ty)]:
        d = np.abs(rng.normal(0.0, 1e-3, nblk)).astype("<f2")
        blocks[:, off : off + 2] = d.view(np.uint8).reshape(nblk, 2)
    return blocks.reshape(-1)


def cpu_child(threads: int, full_sweep: bool) -> dict:
    """Runs in a child process without torch (OMP_PROC_BIND is fixed when OpenMP starts): the reference CPU
    path as this repository's C restatement (oracle/vq_oracle.c: the reference's Cpu_qmv, qwen_cpu.c:581-641,
    bit-identical to it, tests/test_oracle.py) on BASELINE.json configs 1-3 (median of 10 timed calls after one
    warm-up call each) and on config 4: the full 27B sweep (every matrix of the step, 13.4 GiB of distinct
    host memory, one warm-up pass and one timed pass) when full_sweep, else each distinct matrix shape (median
    of 3 calls; the LM head on 1/16 of its rows, scaled) weighted by its per-step count."""
    import statistics

    import numpy as np

    from oracle import oracle
    from vinf_3080ti_amd import synth

    def prepare(ty, w, rows, cols, x, ntok):
        return lambda: oracle.qmv(ty, w, rows, cols, x, ntok, threads=threads)

    def med(fns, reps):
        for f in fns:
            f()
        ts = []
        for _ in range(reps):
            t0 = time.perf_counter()
            for f in fns:
                f()
            ts.append(time.perf_counter() - t0)
        return statistics.median(ts)

    rng = np.random.default_rng(5)
    H, F = 5120, 17408
    res = {}
    w1 = synth.baseline_rows(Q4_K, 4096, 4096, rng)
    x1 = rng.standard_normal(4096).astype(np.float32)
    t = med([prepare(Q4_K, w1, 4096, 4096, x1, 1)], 10)
    res["config1_Q4_K_4096x4096_b1"] = {"ms": t * 1e3, "GBps": alg_bytes(Q4_K, 4096, 4096, 1) / t / 1e9}
    wg, wu = synth.baseline_rows(Q3_K, F, H, rng), synth.baseline_rows(Q3_K, F, H, rng)
    wd = synth.baseline_rows(Q6_K, H, F, rng)
    for n in (1, 4, 8):
        xh, xf = rng.standard_normal(n * H).astype(np.float32), rng.standard_normal(n * F).astype(np.float32)
        fns = [prepare(Q3_K, wg, F, H, xh, n), prepare(Q3_K, wu, F, H, xh, n), prepare(Q6_K, wd, H, F, xf, n)]
        t = med(fns, 10)
        b = 2 * alg_bytes(Q3_K, F, H, n) + alg_bytes(Q6_K, H, F, n)
        res[f"config2_mlp_b{n}"] = {"ms": t * 1e3, "GBps": b / t / 1e9}
    del wg, wu, wd
    for ty in (IQ4_XS, IQ3_S, IQ2_XXS):
        w3 = synth.baseline_rows(ty, H, F, rng)
        for n in (1, 8):
            x3 = rng.standard_normal(n * F).astype(np.float32)
            t = med([prepare(ty, w3, H, F, x3, n)], 10)
            res[f"config3_{TYPE_NAMES[ty]}_{H}x{F}_b{n}"] = {"ms": t * 1e3, "GBps": alg_bytes(ty, H, F, n) / t / 1e9}
    plan = sweep_plan()
    total_b = sum(alg_bytes(ty, rows, cols, 1) for _, ty, rows, cols, _ in plan)
    if full_sweep:
        base = rng.integers(0, 2**63, size=2 << 20, dtype=np.uint64)
        t0 = time.perf_counter()
        mats = [(ty, fast_baseline_rows(ty, rows, cols, rng, base), rows, cols) for _, ty, rows, cols, _ in plan]
        gen_s = time.perf_counter() - t0
        xs = {c: rng.standard_normal(c).astype(np.float32) for c in {m[3] for m in mats}}
        passes = []
        for _ in range(2):
            t0 = time.perf_counter()
            for ty, w, rows, cols in mats:
                oracle.qmv(ty, w, rows, cols, xs[cols], 1, threads=threads)
            passes.append(time.perf_counter() - t0)
        del mats
        res["config4_sweep_b1"] = {"ms": passes[1] * 1e3, "GBps": total_b / passes[1] / 1e9,
                                   "warmup_pass_ms": passes[0] * 1e3, "weights_generated_s": gen_s, "full": 1}
    else:
        counts = {}
        for _, ty, rows, cols, _ in plan:
            counts[(ty, rows, cols)] = counts.get((ty, rows, cols), 0) + 1
        total_s = 0.0
        for (ty, rows, cols), count in counts.items():
            r = rows if rows < 100000 else rows // 16
            w = synth.baseline_rows(ty, r, cols, rng)
            x = rng.standard_normal(cols).astype(np.float32)
            total_s += med([prepare(ty, w, r, cols, x, 1)], 3) * (rows / r) * count
        res["config4_sweep_b1"] = {"ms": total_s * 1e3, "GBps": total_b / total_s / 1e9, "full": 0}
    return {"kind": "port", "threads": threads,
            "configs": {k: {a: round(v, 3) for a, v in d.items()} for k, d in res.items()}}


def cpu_baseline() -> dict:
    """The reference CPU path (its bit-identical C restatement) on the GPU box's host, each setting in a child
    process started before this process touches the GPU: one thread per physical core, bound close
    (OMP_PROC_BIND=close, OMP_PLACES=cores), capped at the GPU's host share of CPU_SHARE CPUs -- the reported
    figure, with the full 27B sweep when the host has FULL_SWEEP_MIN_RAM -- and the reference's default thread
    count omp_get_num_procs() / 2 (qwen_cpu.c:438) on the sampled sweep, for comparison."""
    import subprocess

    host = host_cpu()
    host["ram_bytes"] = host_ram_bytes()
    nprocs = host["cpus_in_affinity"]
    phys = min(host["physical_cores"] or nprocs, nprocs)
    full = host["ram_bytes"] >= FULL_SWEEP_MIN_RAM
    settings = {"all_cores_close": (max(1, min(CPU_SHARE, phys)), {"OMP_PROC_BIND": "close", "OMP_PLACES": "cores"},
                                    full),
                "ref_default": (max(1, min(CPU_SHARE, nprocs // 2)), {}, False)}
    runs = {}
    for label, (threads, extra, sweep_full) in settings.items():
        env = dict(os.environ, **extra, OMP_NUM_THREADS=str(threads))
        cmd = [sys.executable, str(ROOT / "bench.py"), "--cpu-child", str(threads)] + (["--cpu-full"] if sweep_full else [])
        out = subprocess.run(cmd, env=env, capture_output=True, text=True, timeout=900)
        if out.returncode != 0:
            raise RuntimeError(f"cpu baseline child failed: {out.stderr[-2000:]}")
        runs[label] = json.loads(out.stdout.strip().splitlines()[-1])
    main_run = runs["all_cores_close"]
    sweep = main_run["configs"]["config4_sweep_b1"]
    if sweep.get("full"):
        sample = ("the full 27B sweep at batch 1: every matrix of the step once (13.4 GiB of weights in host memory, "
                  "one warm-up pass, then one timed pass)")
    else:
        sample = ("27B sweep at batch 1 estimated from each distinct matrix shape (median of 3 calls, LM head on "
                  f"1/16 of its rows, scaled): host RAM below {FULL_SWEEP_MIN_RAM >> 30} GiB")
    return {"value": sweep["GBps"], "unit": "GB/s", "cores": main_run["threads"], "threads": main_run["threads"],
            "kind": main_run["kind"], "ms_per_step": sweep["ms"], "host": host,
            "sample": sample + "; configs 1-3 timed whole, median of 10 calls after a warm-up call; one thread per "
                      f"physical core, capped at the GPU's host share ({CPU_SHARE})",
            "settings": {k: {"threads": v["threads"], "env": settings[k][1], "configs": v["configs"]}
                         for k, v in runs.items()}}


def stamps_report(torch) -> dict:
    """Per-workgroup timeline of the sweep's streaming launches from the timing build (vinf_3080ti_amd/_var/
    libvq_stamps.so, `python -m vinf_3080ti_amd.build --stamps`): each workgroup's thread 0 stamps s_memrealtime
    (100 MHz, kept in LDS until the end) at entry, when waves 0, 2 and 4 have quantized their activations, at the
    start-up barrier, when wave 0's first weight stage has landed, after every wave's last stage and at the end.
    Launches run one at a time after a producer kernel writes x, rotating over 6 weight copies; medians over 10
    launches."""
    import ctypes

    import numpy as np

    from vinf_3080ti_amd.build import STAMPS_LIB

    lib_path = Path(os.environ.get("VQ_STAMPS_LIB", STAMPS_LIB))  # another timing build, for comparisons
    hip = Hip(torch, lib_path)
    raw = ctypes.CDLL(str(lib_path))
    n = 8192 * 8

    def read(tu):
        buf = np.zeros(n, np.uint64)
        st = getattr(raw, "vq_stamps_read_" + tu)(buf.ctypes.data_as(ctypes.c_void_p), ctypes.c_size_t(n * 8))
        assert st == 0, st
        return buf.reshape(-1, 8).astype(np.int64)

    cases = [("Q3_K gate+up 2x17408x5120", "q3_k", [(Q3_K, 17408, 5120)] * 2, 5120),
             ("Q4_K down 5120x17408", "q4_k", [(Q4_K, 5120, 17408)], 17408),
             ("Q6_K out 5120x6144", "q6_k", [(Q6_K, 5120, 6144)], 6144),
             ("Q4_K 4096x4096 (config 1)", "q4_k", [(Q4_K, 4096, 4096)], 4096)]
    slots = {4: "wave0_activations_quantized", 5: "wave2_activations_quantized", 7: "wave4_activations_quantized",
             1: "startup_barrier",
             6: "wave0_first_stage_landed", 2: "all_waves_loop_done", 3: "end"}
    out = {}
    for name, tu, mats, cols in cases:
        ws = [[make_weights(torch, t, r, c, 100 * k + i)[0] for i, (t, r, c) in enumerate(mats)] for k in range(6)]
        x = torch.randn(1, cols, device="cuda")
        ys = [torch.empty(1, r, device="cuda") for _, r, _ in mats]
        rows = [r for _, r, _ in mats]
        rel, skew, span = [], [], []
        for it in range(14):
            x.mul_(1.0)  # a producer kernel writes x just before, as in a forward pass
            before = read(tu)
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record()
            hip.group_f32(mats[0][0], ws[it % 6], rows, ys, cols, x, 1)
            e1.record()
            torch.cuda.synchronize()
            after = read(tu)
            ch = np.nonzero(after[:, 0] != before[:, 0])[0]
            if it < 4:
                continue
            a = after[ch]
            rel.append((a - a[:, :1]) * 0.01)
            t0 = a[:, 0] - a[:, 0].min()
            b = np.arange(len(ch))
            skew.append([float(t0[b % 8 == k].mean()) * 0.01 for k in range(8)])
            span.append(((a[:, 3].max() - a[:, 0].min()) * 0.01, e0.elapsed_time(e1) * 1e3))
        r = np.concatenate(rel)
        out[name] = {
            "per_workgroup_us_from_its_entry": {v: {"p10": round(float(np.percentile(r[:, k], 10)), 2),
                                                    "median": round(float(np.median(r[:, k])), 2),
                                                    "p90": round(float(np.percentile(r[:, k], 90)), 2)}
                                                for k, v in slots.items()},
            "mean_start_by_blockIdx_mod_8_us": [round(float(np.median([sk[k] for sk in skew])), 2) for k in range(8)],
            "launch_span_first_entry_to_last_end_us": round(float(np.median([s_[0] for s_ in span])), 2),
            "event_us_single_launch": round(float(np.median([s_[1] for s_ in span])), 2),
        }
        log(name, json.dumps(out[name]))
        del ws
        torch.cuda.empty_cache()
    return out


def main() -> None:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=30)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--ntok", type=int, default=1)
    ap.add_argument("--no-graph", action="store_true")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-per-type", action="store_true")
    ap.add_argument("--roofline-only", action="store_true",
                    help="only the dominant launch (plus a 256 MiB device copy that calibrates PMC byte counters)")
    ap.add_argument("--prefill-only", action="store_true",
                    help="only the prefill contraction legs (512 tokens x Q4_K, both shapes)")
    ap.add_argument("--matvec", default="",
                    help="only these matvec launches: comma-separated TYPE:ROWS:COLS[:NTOK[:GROUP[:r]]] "
                         "(e.g. IQ2_XXS:5120:17408:1), timed as the per-type legs are; r: one vq_qmv call "
                         "routed with its workspace (the @batch8 legs)")
    ap.add_argument("--libs", default="",
                    help="with --matvec: comma-separated builds of libvq_hip.so compared launch for launch")
    ap.add_argument("--ops-only", action="store_true",
                    help="only the sequence ops (gated delta, conv update, attention) at the qwen35 shapes")
    ap.add_argument("--mlp-only", action="store_true",
                    help="only the SwiGLU MLP block at batch 1, 4, 8 (as vq_qmv routes) and 8 on the streaming kernel")
    ap.add_argument("--stamps", action="store_true",
                    help="only the per-workgroup timeline of the sweep's streaming launches (needs the timing build: "
                         "python -m vinf_3080ti_amd.build --stamps)")
    ap.add_argument("--cpu-child", type=int, default=0, help=argparse.SUPPRESS)
    ap.add_argument("--cpu-full", action="store_true", help=argparse.SUPPRESS)
    args = ap.parse_args()
    if args.cpu_child:
        print(json.dumps(cpu_child(args.cpu_child, args.cpu_full)), flush=True)
        return
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py measures one GPU: this build has no multi-GPU path (the matvec would shard by weight "
              "rows, one all-gather of y per layer). Run with --gpus 1.", file=sys.stderr)
        sys.exit(2)

    full = not (args.matvec or args.prefill_only or args.mlp_only or args.roofline_only or args.ops_only
                or args.stamps)
    cpu = None
    if full and not args.no_cpu:  # child processes, started before this process initialises the GPU
        log("cpu baseline: reference CPU path (C restatement), configs 1-3 and the 27B sweep, two thread settings")
        cpu = cpu_baseline()

    import torch

    assert torch.cuda.is_available(), "bench.py needs a GPU"
    if args.stamps:
        print(json.dumps({"stamps": stamps_report(torch)}), flush=True)
        return
    hip = Hip(torch)

    if args.matvec and args.libs:
        hips = [Hip(torch, p) for p in args.libs.split(",")]
        from vinf_3080ti_amd import GGUFTensorType

        by_name = {t.name: int(t) for t in GGUFTensorType}
        out = {}
        for spec in args.matvec.split(","):
            f = spec.split(":")
            ntok = int(f[3]) if len(f) > 3 else 1
            group = int(f[4]) if len(f) > 4 else 1
            r = ab_matvec(torch, hips, by_name[f[0]], int(f[1]), int(f[2]), ntok, group)
            out[spec] = dict(zip(args.libs.split(","), r))
            log(spec + ": " + "  ".join(f"{Path(p).stem} {v['med_us']} (min {v['min_us']})" for p, v in out[spec].items()))
        print(json.dumps({"ab": out}), flush=True)
        return
    if args.matvec:
        out = {}
        from vinf_3080ti_amd import GGUFTensorType

        by_name = {t.name: int(t) for t in GGUFTensorType}
        for spec in args.matvec.split(","):
            f = spec.split(":")
            ty, rows, cols = by_name[f[0]], int(f[1]), int(f[2])
            ntok = int(f[3]) if len(f) > 3 else 1
            group = int(f[4]) if len(f) > 4 else 1
            if len(f) > 5 and f[5] == "r":  # routed: one vq_qmv call with its workspace, as a caller gets it
                r = bench_matvec_routed(torch, hip, ty, rows, cols, ntok, iters=100)
            else:
                r = bench_matvec(torch, hip, ty, rows, cols, ntok, iters=100, group=group)
            out[spec] = {k: round(v, 4) if isinstance(v, float) else v for k, v in r.items()}
            log(f"{spec}: {out[spec]['us']} us, {out[spec]['GBps']} GB/s")
        print(json.dumps({"matvec": out}), flush=True)
        return
    if args.ops_only:
        print(json.dumps({"ops": bench_ops(torch, hip)}), flush=True)
        return
    if args.prefill_only:
        out = {}
        for rows, cols in ((17408, 5120), (5120, 17408)):
            out[f"Q4_K_{rows}x{cols}_M512"] = bench_gemm(torch, hip, Q4_K, rows, cols, 512)
        # The other types of a UD-Q3_K_XL prompt pass: FFN gate/up (Q3_K), attention/SSM projections (Q5_K, Q6_K);
        # and the FFN gate/up of Q2_K-, IQ2- and IQ3_XXS-based mixes.
        for ty, rows, cols in ((Q3_K, 17408, 5120), (Q6_K, 5120, 17408), (Q5_K, 10240, 5120), (Q6_K, 5120, 6144),
                               (Q2_K, 17408, 5120), (IQ2_XS, 17408, 5120), (IQ2_XXS, 17408, 5120),
                               (IQ2_S, 17408, 5120), (IQ3_XXS, 17408, 5120)):
            out[f"{TYPE_NAMES[ty]}_{rows}x{cols}_M512"] = bench_gemm(torch, hip, ty, rows, cols, 512)
        # The reference's own numerics (activations rounded to f16): vq_qgemm_f16x_ws.
        for ty, rows, cols in ((Q4_K, 17408, 5120), (Q4_K, 5120, 17408), (Q3_K, 17408, 5120), (Q6_K, 5120, 17408),
                               (Q5_K, 10240, 5120), (Q6_K, 5120, 6144), (Q2_K, 17408, 5120), (IQ2_XS, 17408, 5120),
                               (IQ2_XXS, 17408, 5120), (IQ2_S, 17408, 5120), (IQ3_XXS, 17408, 5120)):
            out[f"{TYPE_NAMES[ty]}_{rows}x{cols}_M512_f16x"] = bench_gemm(torch, hip, ty, rows, cols, 512, f16x=True)
        print(json.dumps({"prefill": out}), flush=True)
        return
    if args.mlp_only:
        out = {f"batch{n}": bench_mlp(torch, hip, n) for n in (1, 4, 8)}
        out["batch8_stream"] = bench_mlp(torch, hip, 8, mfma=False)
        print(json.dumps({"mlp_block": out}), flush=True)
        return

    # Roofline of the dominant kernel: the FFN gate+up launch (2 x Q3_K 17408x5120, 64 launches per step).
    log("roofline: grouped Q3_K 2 x 17408x5120 matvec")
    dom = bench_matvec(torch, hip, Q3_K, 17408, 5120, args.ntok, iters=100, group=2, reps=5)
    traffic = profiled_traffic()
    trace_us = profiled_trace_us()
    roofline = {
        "bound": "hbm",
        "kernel": f"qmv_stream_kernel<Q3_K,{args.ntok}> gate+up group 2x17408x5120",
        "achieved": round(dom["GBps"], 2),
        "peak": HBM_PEAK_GBPS,
        "unit": "GB/s",
        "frac": round(dom["frac"], 4),
        "avg_us": round(dom["us"], 3),
        "traffic": traffic,
        # not counted in this run: the committed rocprofv3 summaries of the same launch and command
        "traffic_source": "profiles/qmv_q3k_gateup_2x17408x5120_pmc.md (rocprofv3 FETCH_SIZE / WRITE_SIZE)",
        "trace_avg_us": trace_us,
        "trace_frac": round(dom["bytes"] / (trace_us * 1e-6) / 1e9 / HBM_PEAK_GBPS, 4) if trace_us else None,
        "trace_source": "profiles/qmv_q3k_gateup_2x17408x5120_pmc.md (rocprofv3 --kernel-trace of bench.py "
                        "--roofline-only: the kernel's own duration, without the graph's launch gaps)",
    }
    if args.roofline_only:
        a = torch.empty(256 << 20, dtype=torch.uint8, device="cuda")
        b = torch.empty_like(a)
        for _ in range(3):
            b.copy_(a)  # PMC calibration: 256 MiB read + 256 MiB written per copy
        torch.cuda.synchronize()
        print(json.dumps({"roofline": roofline, "bytes_per_launch": dom["bytes"]}), flush=True)
        return
    per_type = {}
    if not args.no_per_type:
        for ty in PER_TYPE:
            log(f"per-type: {TYPE_NAMES[ty]} 5120x17408")
            r = bench_matvec(torch, hip, ty, 5120, 17408, args.ntok, reps=3)  # median of 3 graph replays
            per_type[TYPE_NAMES[ty]] = {k: round(v, 4) if isinstance(v, float) else v for k, v in r.items()}
        r = bench_matvec(torch, hip, Q4_K, 4096, 4096, args.ntok, reps=3)
        per_type["Q4_K@4096x4096"] = {k: round(v, 4) if isinstance(v, float) else v for k, v in r.items()}
        for ty in (IQ4_XS, IQ3_S, IQ2_XXS):  # config 3 at batch 8, routed as vq_qmv routes it
            log(f"per-type batch 8: {TYPE_NAMES[ty]} 5120x17408")
            per_type[f"{TYPE_NAMES[ty]}@batch8"] = bench_matvec_routed(torch, hip, ty, 5120, 17408, 8)

    prefill, mlp, ops = {}, {}, {}
    if not args.no_per_type:
        for n in (1, 4, 8):
            log(f"SwiGLU MLP block, batch {n}")
            mlp[f"batch{n}"] = bench_mlp(torch, hip, n)
        mlp["batch8_stream"] = bench_mlp(torch, hip, 8, mfma=False)
        for rows, cols in ((17408, 5120), (5120, 17408)):
            log(f"prefill: 512 tokens x Q4_K {rows}x{cols}")
            prefill[f"Q4_K_{rows}x{cols}_M512"] = bench_gemm(torch, hip, Q4_K, rows, cols, 512)
            # the reference's numerics for this config (fp16 activations, one MFMA per product)
            prefill[f"Q4_K_{rows}x{cols}_M512_f16x"] = bench_gemm(torch, hip, Q4_K, rows, cols, 512, f16x=True)
        log("sequence ops (gated delta, conv update, attention)")
        ops = bench_ops(torch, hip)

    log("sweep: allocating 13.4 GiB of weights")
    sw = Sweep(torch, hip, args.ntok)
    for _ in range(args.warmup):
        sw.step()
    torch.cuda.synchronize()
    graph = None
    if not args.no_graph:
        graph = torch.cuda.CUDAGraph()
        s = torch.cuda.Stream()
        s.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(s):
            with torch.cuda.graph(graph, stream=s):
                sw.step()
        torch.cuda.synchronize()
        for _ in range(args.warmup):
            graph.replay()
        torch.cuda.synchronize()
    log(f"sweep: timing {args.steps} steps ({'graph' if graph else 'eager'})")
    start, stop = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    start.record()
    for _ in range(args.steps):
        graph.replay() if graph else sw.step()
    stop.record()
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    ms = start.elapsed_time(stop) / args.steps
    value = sw.bytes / (ms * 1e-3) / 1e9

    sweep4 = None
    if not args.no_per_type and args.ntok == 1:
        log("sweep at batch 4 (same resident weights)")
        sw4 = Sweep(torch, hip, 4, weights=sw.w)
        ms4, _ = time_sweep(torch, sw4, max(5, args.steps // 3), args.warmup, use_graph=not args.no_graph)
        sweep4 = {"ms_per_step": round(ms4, 4), "GBps": round(sw4.bytes / (ms4 * 1e-3) / 1e9, 2),
                  "frac": round(sw4.bytes / (ms4 * 1e-3) / 1e9 / HBM_PEAK_GBPS, 4)}
        del sw4

    out = {
        "metric": METRIC,
        "value": round(value, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int8",
        "data": "synthetic",
        "config": {
            "workload": f"qwen35-27B decode-step weight sweep (UD-Q3_K_XL-like mix, Q6_K LM head + argmax), batch {args.ntok}",
            "ntok": args.ntok,
            "bytes_per_step": sw.bytes,
            "weight_bytes_per_step": sw.weight_bytes,
            "launch": "hipGraph" if graph else "eager",
            "launches_per_step": sw.launches,
            "frac_of_hbm_peak": round(value / HBM_PEAK_GBPS, 4),
            "wall_s": round(wall, 3),
        },
        "roofline": roofline,
        "cpu_baseline": None if cpu is None else {k: (round(v, 3) if isinstance(v, float) else v) for k, v in cpu.items()},
        "per_type": per_type,
        "prefill": prefill,
        "mlp_block": mlp,
        "ops": ops,
        "sweep_batch4": sweep4,
    }
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
