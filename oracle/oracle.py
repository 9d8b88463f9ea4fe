"""ctypes binding of oracle/libvq_oracle.so (test infrastructure only; see vq_oracle.c's header).

Functions mirror the reference CPU path (/root/reference/engine/csrc/cpu/qwen_cpu.c):
  qmv            Cpu_qmv (:581-641) with dot_row_q/dot_row_f (:125-360), bit-identical fp32 outputs
  quantize_x     activation quantizer (:607-627)
  dequant_rows   dequant.py:121-500 / qwen_quant.cuh deq8 (:151-279)
  int_partials   exact int32 sum of code*xq per (token, row, group, 16-half)
  decode_codes   integer codes + per-16 scales/mins with dequant == scale*code - min
  qgemm_f16x     prompt GEMM with fp16 activations (f32_to_f16_rows_kernel + vinf_qgemm_kernel,
                 qwen_runtime.cu:657-739), exact weights, float64 numpy
  argmax_rows    argmax_kernel (qwen_runtime.cu:850-876), ties to the lowest index
  stage_x        the megakernel's QMV activation staging (qwen_megakernel.cu:485-551), float64 numpy
  rope_neox      NeoX partial RoPE (rope_neox_kernel, qwen_runtime.cu:81-92), float64 numpy
  attention      GQA attention with causal / bidirectional / window visibility (qwen_runtime.cu:128-162)
  conv_update    causal depthwise conv + SiLU state stepping (conv_update_kernel, qwen_runtime.cu:401-426)
  gated_delta    gated delta rule state stepping (gated_delta_kernel, qwen_runtime.cu:515-567)
"""
from __future__ import annotations

import ctypes
import os
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
LIB_PATH = HERE / "libvq_oracle.so"

_TABLE_IDS = {"iq2xxs_grid": 0, "iq2xs_grid": 1, "iq2s_grid": 2, "iq3xxs_grid": 3, "iq3s_grid": 4, "ksigns_iq2xs": 5}

_lib = None


def build() -> None:
    import subprocess

    subprocess.check_call(["make", "-s", "-C", str(HERE), "all"])


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            build()
        L = ctypes.CDLL(str(LIB_PATH))
        P, I = ctypes.c_void_p, ctypes.c_int
        L.vqo_traits.argtypes = [I, ctypes.POINTER(I), ctypes.POINTER(I)]
        L.vqo_table.argtypes = [I, P]
        L.vqo_dequant_rows.argtypes = [I, P, I, I, P]
        L.vqo_decode_codes.argtypes = [I, P, I, I, P, P, P]
        L.vqo_quantize_x.argtypes = [P, I, I, P, P, P]
        L.vqo_int_partials.argtypes = [I, P, I, I, P, I, P]
        L.vqo_qmv.argtypes = [I, P, I, I, P, I, P, I]
        L.vqo_argmax_rows.argtypes = [P, I, I, P]
        _lib = L
    return _lib


def _p(a: np.ndarray) -> int:
    assert a.flags["C_CONTIGUOUS"]
    return a.ctypes.data


def _u8(raw) -> np.ndarray:
    return np.ascontiguousarray(np.frombuffer(raw, dtype=np.uint8) if isinstance(raw, (bytes, bytearray, memoryview)) else raw, dtype=np.uint8)


def traits(type_id: int) -> tuple[int, int]:
    bs, ts = ctypes.c_int(), ctypes.c_int()
    if not lib().vqo_traits(type_id, ctypes.byref(bs), ctypes.byref(ts)):
        raise ValueError(f"unsupported type {type_id}")
    return bs.value, ts.value


def table(name: str) -> bytes:
    n = lib().vqo_table(_TABLE_IDS[name], None)
    buf = np.empty(n, np.uint8)
    lib().vqo_table(_TABLE_IDS[name], _p(buf))
    return buf.tobytes()


def dequant_rows(type_id: int, raw, rows: int, cols: int) -> np.ndarray:
    w = _u8(raw)
    out = np.empty((rows, cols), np.float32)
    if lib().vqo_dequant_rows(type_id, _p(w), rows, cols, _p(out)):
        raise ValueError("dequant_rows: bad type/shape")
    return out


def decode_codes(type_id: int, raw, rows: int, cols: int):
    w = _u8(raw)
    codes = np.empty((rows, cols), np.int8)
    scales = np.empty((rows, cols // 16), np.float32)
    mins = np.empty((rows, cols // 16), np.float32)
    if lib().vqo_decode_codes(type_id, _p(w), rows, cols, _p(codes), _p(scales), _p(mins)):
        raise ValueError("decode_codes: bad type/shape")
    return codes, scales, mins


def quantize_x(x: np.ndarray, ntok: int, cols: int):
    x = np.ascontiguousarray(x, np.float32).reshape(ntok, cols)
    xq = np.empty((ntok, cols), np.int8)
    xd = np.empty((ntok, cols // 32), np.float32)
    xs = np.empty((ntok, cols // 32), np.float32)
    if lib().vqo_quantize_x(_p(x), ntok, cols, _p(xq), _p(xd), _p(xs)):
        raise ValueError("quantize_x: bad shape")
    return xq, xd, xs


def int_partials(type_id: int, raw, rows: int, cols: int, xq: np.ndarray, ntok: int) -> np.ndarray:
    w = _u8(raw)
    xq = np.ascontiguousarray(xq, np.int8)
    out = np.empty((ntok, rows, cols // 32, 2), np.int32)
    if lib().vqo_int_partials(type_id, _p(w), rows, cols, _p(xq), ntok, _p(out)):
        raise ValueError("int_partials: bad type/shape")
    return out


def qmv(type_id: int, raw, rows: int, cols: int, x: np.ndarray, ntok: int, threads: int | None = None) -> np.ndarray:
    w = _u8(raw)
    x = np.ascontiguousarray(x, np.float32).reshape(ntok, cols)
    y = np.empty((ntok, rows), np.float32)
    if threads is None:
        threads = os.cpu_count() or 1
    if lib().vqo_qmv(type_id, _p(w), rows, cols, _p(x), ntok, _p(y), threads):
        raise ValueError("qmv: bad type/shape")
    return y


def f16x_scales(x: np.ndarray) -> np.ndarray:
    """Per token 2^min(15 - E, 126) with max|x| < 2^E (frexp), 1 for an all-zero token: the largest scaled |x| lies
    in [2^14, 2^15), far inside fp16's range."""
    m = np.abs(x).max(axis=1).astype(np.float64)
    e = np.frexp(m)[1]
    return np.where(m > 0, np.ldexp(1.0, np.minimum(15 - e, 126)), 1.0)


def f16x_weights(type_id: int, raw, rows: int, cols: int) -> np.ndarray:
    """The weights of the f16-activation contraction, float64: exact (dequant_rows) for every type but Q6_K, whose
    integer product (q - 32) sc (up to 32 x 128, past fp16's exact integers) is rounded to fp16 once before d
    applies: d f16((q - 32) sc), within 2^-11 of the exact weight, as the reference rounds every dequantized weight
    to fp16 (vinf_qgemm_kernel's a_tile, qwen_runtime.cu:700-702). Q6_K block: ql[128] qh[64] scales[16] int8
    d f16 (210 bytes); scale j covers elements 16 j .. 16 j + 15."""
    exact = dequant_rows(type_id, raw, rows, cols).astype(np.float64)
    if type_id != 14:
        return exact
    codes, _, _ = decode_codes(type_id, raw, rows, cols)
    blk = _u8(raw)[: rows * (cols // 256) * 210].reshape(rows, cols // 256, 210)
    sc = blk[:, :, 192:208].copy().view(np.int8).astype(np.float64).reshape(rows, cols // 16)
    d = blk[:, :, 208:210].copy().view(np.float16).astype(np.float64).reshape(rows, cols // 256)
    prod = codes.astype(np.float64).reshape(rows, cols // 16, 16) * sc[:, :, None]
    w = prod.astype(np.float16).astype(np.float64).reshape(rows, cols // 256, 256) * d[:, :, None]
    return w.reshape(rows, cols)


def qgemm_f16x(type_id: int, raw, rows: int, cols: int, x: np.ndarray, ntok: int) -> np.ndarray:
    """y[t] = W f16(x[t] s_t) / s_t in float64: W = f16x_weights (exact, Q6_K rounded once), f16 the IEEE
    round-to-nearest-even conversion the reference applies to every activation before its fp16 MMA
    (f32_to_f16_rows_kernel, qwen_runtime.cu:657-661; vinf_qgemm_kernel :663-739 accumulates the products in fp32),
    s_t = f16x_scales. Scaling by a power of two commutes with the rounding wherever x s_t and x are both normal
    fp16 numbers, so for such tokens this is W f16(x) exactly."""
    w = f16x_weights(type_id, raw, rows, cols)
    x = np.ascontiguousarray(x, np.float32).reshape(ntok, cols)
    s = f16x_scales(x)
    xb = (x * s[:, None].astype(np.float32)).astype(np.float16).astype(np.float64)
    return (xb @ w.T) / s[:, None]


def argmax_rows(x: np.ndarray, n: int, ntok: int) -> list[int]:
    x = np.ascontiguousarray(x, np.float32).reshape(ntok, n)
    out = np.empty(ntok, np.int32)
    lib().vqo_argmax_rows(_p(x), n, ntok, _p(out))
    return [int(v) for v in out]


# Activation staging flags (runtime/instructions.py:179-182).
STAGE_ADD, STAGE_NORM, STAGE_SILU_MUL = 1, 2, 8


def stage_x(x: np.ndarray, x2: np.ndarray | None, norm_w: np.ndarray | None, eps: float, flags: int) -> np.ndarray:
    """float64 restatement of op_qmv's staging (qwen_megakernel.cu:485-551): v = silu(x) * x2 with SILU_MUL
    (silu(z) = z / (1 + exp(-z)), silu_f), then with NORM v * norm_w / sqrt(mean(v^2) + eps) per token (the
    megakernel's rsqrtf(block_sum(v^2) / cols + eps), :500)."""
    v = np.asarray(x, np.float64).copy()
    if flags & STAGE_SILU_MUL:
        v = v / (1.0 + np.exp(-v)) * np.asarray(x2, np.float64)
    if flags & STAGE_NORM:
        ms = (v * v).mean(axis=-1, keepdims=True)
        v = v / np.sqrt(ms + eps) * np.asarray(norm_w, np.float64)
    return v


def rope_neox(x: np.ndarray, heads: int, hd: int, rot: int, pos0: int, base: float) -> np.ndarray:
    """float64 NeoX RoPE of x [ntok][heads][hd] (rope_neox_kernel, qwen_runtime.cu:81-92): for j < rot/2 the
    pair (x[j], x[j + rot/2]) of token t turns by (pos0 + t) * base^(-2j/rot); dims >= rot are untouched."""
    v = np.array(x, np.float64).reshape(-1, heads, hd)
    half = rot // 2
    j = np.arange(half)
    ang = (pos0 + np.arange(v.shape[0]))[:, None] * base ** (-2.0 * j / rot)[None, :]
    c, s = np.cos(ang)[:, None, :], np.sin(ang)[:, None, :]
    a, b = v[..., :half].copy(), v[..., half:rot].copy()
    v[..., :half] = a * c - b * s
    v[..., half:rot] = b * c + a * s
    return v


def attention(q: np.ndarray, kc: np.ndarray, vc: np.ndarray, heads: int, kv_heads: int, seq_len: int,
              bidirectional: bool = False, window: int = 0) -> np.ndarray:
    """float64 GQA attention (attention_kernel, qwen_runtime.cu:128-162): q [ntok][heads][hd], caches
    [kv_heads][max_seq][hd]; token t sees positions [start, seq_len + t) (causal) or [start, seq_len + ntok - 1)
    (bidirectional), start = seq_len + t - window when window > 0 and positive; scores scaled by 1/sqrt(hd)."""
    q = np.asarray(q, np.float64)
    ntok, _, hd = q.shape
    out = np.zeros_like(q)
    for t in range(ntok):
        qend = seq_len + t
        end = seq_len + ntok - 1 if bidirectional else qend
        start = qend - window if window > 0 and qend > window else 0
        for h in range(heads):
            kvh = h // (heads // kv_heads)
            k = np.asarray(kc[kvh, start:end], np.float64)
            v = np.asarray(vc[kvh, start:end], np.float64)
            s = k @ q[t, h] / np.sqrt(hd)
            p = np.exp(s - s.max())
            out[t, h] = (p / p.sum()) @ v
    return out


def conv_update(x: np.ndarray, state: np.ndarray, w: np.ndarray):
    """float64 conv_update_kernel (qwen_runtime.cu:401-426): x [ntok][channels], state and w [channels][K].
    Returns (out [ntok][channels], final state, snapshots [ntok - 1][channels][K])."""
    st = np.array(state, np.float64)
    w = np.asarray(w, np.float64)
    outs, snaps = [], []
    for t, xt in enumerate(np.asarray(x, np.float64)):
        st = np.concatenate([st[:, 1:], xt[:, None]], axis=1)
        a = (st * w).sum(axis=1)
        outs.append(a / (1.0 + np.exp(-a)))
        if t < len(x) - 1:
            snaps.append(st.copy())
    return np.array(outs), st, np.array(snaps).reshape(-1, *st.shape)


def gated_delta(conv, b, a, ssm_a, dt, state, key_heads: int, value_heads: int, kd: int, vd: int, eps: float,
                head_order: int):
    """float64 gated_delta_kernel (qwen_runtime.cu:515-567). conv [ntok][2 kh kd + vh vd], b / a [ntok][vh],
    ssm_a / dt [vh], state [vh][kd][vd]. Returns (out [ntok][vh][vd], final state, snapshots [ntok - 1])."""
    S = np.array(state, np.float64).reshape(value_heads, kd, vd)
    conv = np.asarray(conv, np.float64)
    outs, snaps = [], []
    for t in range(conv.shape[0]):
        o = np.zeros((value_heads, vd))
        for h in range(value_heads):
            kh = h // (value_heads // key_heads) if head_order == 0 else h % key_heads
            q = conv[t, kh * kd:(kh + 1) * kd]
            k = conv[t, (key_heads + kh) * kd:(key_heads + kh + 1) * kd]
            v = conv[t, 2 * key_heads * kd + h * vd:2 * key_heads * kd + (h + 1) * vd]
            qh = q / (np.sqrt(q @ q + eps) * np.sqrt(kd))
            kh_ = k / np.sqrt(k @ k + eps)
            beta = 1.0 / (1.0 + np.exp(-float(b[t][h])))
            xa = float(a[t][h]) + float(dt[h])
            sp = xa if xa > 20.0 else np.log1p(np.exp(xa))
            S[h] *= np.exp(float(ssm_a[h]) * sp)
            delta = (v - kh_ @ S[h]) * beta
            S[h] += np.outer(kh_, delta)
            o[h] = qh @ S[h]
        outs.append(o)
        if t < conv.shape[0] - 1:
            snaps.append(S.copy())
    return np.array(outs), S, np.array(snaps).reshape(-1, value_heads, kd, vd)


def paged_rows(pt_row, page_size: int, kv_heads: int, kvh: int, positions) -> np.ndarray:
    """Rows of a paged KV pool [page][kv_head][page_size][hd] (viewed as [page * kv_heads * page_size] rows)
    that hold kv head kvh at the given positions of a sequence whose page ids are pt_row (KvAddr::row, qwen_runtime.cu:
    100-110): page pt_row[pos // page_size], slot pos % page_size."""
    pos = np.asarray(positions, np.int64)
    pg = np.asarray(pt_row, np.int64)[pos // page_size]
    return (pg * kv_heads + kvh) * page_size + pos % page_size


def gather_paged(pool: np.ndarray, pt_row, page_size: int, kv_heads: int, length: int) -> np.ndarray:
    """The first `length` positions of one sequence of a paged pool as a contiguous cache [kv_heads][length][hd]."""
    hd = pool.shape[-1]
    flat = pool.reshape(-1, hd)
    return np.stack([flat[paged_rows(pt_row, page_size, kv_heads, h, np.arange(length))] for h in range(kv_heads)])
