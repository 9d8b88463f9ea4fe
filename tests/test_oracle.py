"""Pins of the CPU oracle (oracle/vq_oracle.c) against the reference: KATs from the reference's own tests,
golden vectors written from the reference's compiled CPU path, codebook digests, and exact integer
brute force. CPU only."""
from __future__ import annotations

import glob
import hashlib
import importlib.util
import struct

import numpy as np
import pytest

from conftest import REFERENCE, ROOT
from vinf_3080ti_amd import GGUFTensorType as T
from vinf_3080ti_amd import QUANT_TYPES, synth, tables

ALL_TYPES = list(QUANT_TYPES) + [T.F32, T.F16]


def dq(oracle, ty, block: bytes, cols: int) -> list[float]:
    return [float(v) for v in oracle.dequant_rows(int(ty), block, 1, cols)[0]]


def qs_pair() -> bytes:
    return bytes(lo | (hi << 4) for lo, hi in zip(range(16), reversed(range(16))))


# ---- known-answer tests of the reference (engine/tests/test_gguf_dequant.py) -------------------------

def test_kat_q8_0(oracle_mod):  # test_gguf_dequant.py:38-44
    v = dq(oracle_mod, T.Q8_0, struct.pack("<e32b", 0.5, *range(-16, 16)), 32)
    assert v[0] == -8.0 and v[-1] == 7.5


def test_kat_q4_k(oracle_mod):  # :54-74
    block = struct.pack("<ee", 0.5, 0.25) + bytes([1, 2, 3, 4, 0, 1, 2, 3, 5, 6, 7, 8]) + qs_pair() * 8
    v = dq(oracle_mod, T.Q4_K, block, 256)
    assert v[:4] == [0.0, 0.5, 1.0, 1.5] and v[16:20] == [0.0, 0.5, 1.0, 1.5]
    assert v[32:34] == [14.75, 13.75]
    assert (v[64], v[96], v[128], v[160], v[192], v[224]) == (-0.5, 29.25, 0.0, 45.0, 0.0, 60.0)


def test_kat_q3_k(oracle_mod):  # :76-97
    hmask = bytearray([0xFF] * 32)
    hmask[3] &= ~(1 << 5) & 0xFF
    qs = bytearray([0xFF] * 64)
    qs[32] = 0
    scales = bytes(k | (k + 8) << 4 for k in range(8)) + bytes([0xE4] * 4)
    v = dq(oracle_mod, T.Q3_K, bytes(hmask) + bytes(qs) + scales + struct.pack("<e", 0.5), 256)
    expect = {0: -48.0, 3: -48.0, 35: -45.0, 80: -16.5, 128: 0.0, 129: 12.0, 160: 0.0, 163: -5.0, 255: 46.5}
    assert {k: v[k] for k in expect} == expect


def test_kat_iq3_s_grid():  # :99-106
    g = tables.table("iq3s_grid")
    assert len(g) == 2048
    assert tuple(g[0:4]) == (1, 1, 1, 1) and tuple(g[12:16]) == (11, 1, 1, 1) and tuple(g[20:24]) == (1, 3, 1, 1)


def test_kat_q2_k(oracle_mod):  # :108-125, expected values in ggml's loop order
    scales = bytes((k % 16) | (((7 * k) % 16) << 4) for k in range(16))
    qs = bytes((i * 37 + 11) % 256 for i in range(64))
    v = dq(oracle_mod, T.Q2_K, scales + qs + struct.pack("<ee", 0.5, 0.25), 256)
    expected, idx = [], 0
    for n in range(2):
        q = qs[32 * n : 32 * n + 32]
        for j in range(4):
            for s in range(2):
                sc = scales[idx]
                idx += 1
                expected += [0.5 * (sc & 0xF) * ((q[16 * s + l] >> (2 * j)) & 3) - 0.25 * (sc >> 4) for l in range(16)]
    assert v == [float(np.float32(e)) for e in expected]


def test_kat_q5_k(oracle_mod):  # :127-142
    block = struct.pack("<ee", 0.5, 0.25) + bytes([1, 2, 3, 4, 0, 1, 2, 3, 5, 6, 7, 8]) + bytes([0b01010101] * 32) + qs_pair() * 8
    v = dq(oracle_mod, T.Q5_K, block, 256)
    assert v[:4] == [8.0, 8.5, 9.0, 9.5] and v[32:36] == [14.75, 13.75, 12.75, 11.75]
    assert (v[64], v[96], v[128], v[160], v[192], v[224]) == (23.5, 29.25, 40.0, 45.0, 56.0, 60.0)


def test_kat_q6_k(oracle_mod):  # :144-159
    block = bytes([0x10] * 128) + bytes([0b11100100] * 64) + struct.pack("<16b", *range(1, 17)) + struct.pack("<e", 0.5)
    v = dq(oracle_mod, T.Q6_K, block, 256)
    assert [v[i] for i in range(0, 128, 16)] == [-16.0, -32.0, -24.0, -32.0, 2.5, 3.0, 59.5, 68.0]


def test_kat_iq4_nl(oracle_mod):  # :161-167
    v = dq(oracle_mod, T.IQ4_NL, struct.pack("<e", 0.5) + qs_pair(), 32)
    assert v[:4] == [-63.5, -52.0, -41.5, -32.5] and v[16:20] == [56.5, 44.5, 34.5, 26.5]


def test_kat_iq4_xs(oracle_mod):  # :169-178
    v = dq(oracle_mod, T.IQ4_XS, struct.pack("<eH", 0.5, 0xAAAA) + bytes([0x11] * 4) + qs_pair() * 8, 256)
    assert v[:4] == [-63.5, -52.0, -41.5, -32.5] and v[32:36] == [-63.5, -52.0, -41.5, -32.5]


def test_kat_iq3_s(oracle_mod):  # :180-193
    block = struct.pack("<e", 0.5) + bytes(64) + bytes(8) + bytes([1] + [0] * 31) + bytes(4)
    v = dq(oracle_mod, T.IQ3_S, block, 256)
    assert v[0] == -0.5 and v[1:4] == [0.5, 0.5, 0.5] and v[32] == 0.5


def test_kat_iq2_iq3xxs_closed_form(oracle_mod):
    """No reference KAT covers these four types; pin one hand-built block each from the ggml layout."""
    g2 = tables.table("iq2xxs_grid")
    # IQ2_XXS, d = 1: group 0 picks entries 1,2,3,4 with sign patterns ksigns[1], 0, 0, 0 and scale nibble 15.
    aux0 = 1 | (2 << 8) | (3 << 16) | (4 << 24)
    aux1 = 1 | (15 << 28)
    block = struct.pack("<e", 1.0) + struct.pack("<II", aux0, aux1) + bytes(56)
    v = dq(oracle_mod, T.IQ2_XXS, block, 256)
    db = (0.5 + 15) * 0.25
    ks1 = tables.table("ksigns_iq2xs")[1]  # 0x81: elements 0 and 7 negative
    assert ks1 == 0x81
    first = [db * g2[8 + j] * (-1 if (ks1 >> j) & 1 else 1) for j in range(8)]
    assert v[:8] == first and v[8:16] == [db * g2[16 + j] for j in range(8)]
    assert v[32:40] == [0.5 * 0.25 * 8.0] * 8  # group 1: entry 0 (all 8), scale nibble 0
    # IQ3_XXS, d = 2: group 0 entries (5, 6), sign index 0, scale nibble 3 -> db = 2*(3.5)*0.5
    g3 = tables.table("iq3xxs_grid")
    block = struct.pack("<e", 2.0) + bytes([5, 6]) + bytes(62) + struct.pack("<I", 3 << 28) + bytes(28)
    v = dq(oracle_mod, T.IQ3_XXS, block, 256)
    assert v[:8] == [3.5 * g3[20 + j] for j in range(4)] + [3.5 * g3[24 + j] for j in range(4)]


# ---- codebooks -------------------------------------------------------------------------------------------

@pytest.mark.parametrize("name", ["iq2xxs_grid", "iq2xs_grid", "iq2s_grid", "iq3xxs_grid", "iq3s_grid", "ksigns_iq2xs"])
def test_codebooks_match_reference_digest(golden, oracle_mod, name):
    assert hashlib.sha256(tables.table(name)).digest() == golden[f"sha256_{name}"].tobytes()
    assert oracle_mod.table(name) == tables.table(name)


@pytest.mark.skipif(not REFERENCE.exists(), reason="reference checkout not mounted")
def test_codebooks_match_reference_text():
    import sys

    sys.path.insert(0, str(ROOT / "vinf_3080ti_amd" / "csrc"))
    from gen_iq_grids import reference_tables

    for name, data in reference_tables(REFERENCE.parent).items():
        assert tables.table(name) == data, name


# ---- golden vectors from the reference's compiled CPU path ---------------------------------------------

@pytest.mark.parametrize("ty", ALL_TYPES, ids=lambda t: t.name)
def test_qmv_bit_identical_to_reference_golden(golden, oracle_mod, ty):
    w, x, y = golden[f"w_{ty.name}"], golden[f"x_{ty.name}"], golden[f"y_{ty.name}"]
    got = oracle_mod.qmv(int(ty), w, y.shape[1], x.shape[1], x, x.shape[0], threads=2)
    assert np.array_equal(got.view(np.uint32), y.view(np.uint32))


@pytest.mark.parametrize("ty", QUANT_TYPES, ids=lambda t: t.name)
def test_dequant_matches_reference_one_hot_probe(golden, oracle_mod, ty):
    """probe[c][r] is the reference's qmv of one-hot x = e_c: W[r][c] up to ~3 ulp of activation rounding."""
    w, probe = golden[f"pw_{ty.name}"], golden[f"probe_{ty.name}"].astype(np.float64)
    rows, cols = probe.shape[1], probe.shape[0]
    v = oracle_mod.dequant_rows(int(ty), w, rows, cols).astype(np.float64).T
    _, scales, mins = oracle_mod.decode_codes(int(ty), w, rows, cols)
    mag = np.abs(v) + np.repeat(np.abs(mins).astype(np.float64), 16, axis=1).T
    assert np.all(np.abs(probe - v) <= 2.0**-20 * mag + 1e-30)
    # the probe separates neighbouring codes: the smallest nonzero scale step is far above the tolerance
    assert np.all(2.0**-20 * mag < np.repeat(np.abs(scales).astype(np.float64), 16, axis=1).T + (scales == 0).repeat(16, 1).T)


def test_quantizer_matches_reference_q8_0(golden, oracle_mod):
    """The reference's quantize_q8_0 (qwen_cpu.c:953-985) applies the same amax/127, lrintf rule."""
    for n in range(4):
        x = golden[f"q8x_{n}"]
        blocks = golden[f"q8_{n}"].reshape(-1, 34)
        xq, xd, _ = oracle_mod.quantize_x(x, 1, x.size)
        assert np.array_equal(xq.reshape(-1, 32).view(np.uint8), blocks[:, 2:])
        assert np.array_equal(xd.reshape(-1).astype("<f2").view(np.uint8).reshape(-1, 2), blocks[:, :2])


@pytest.mark.skipif(not glob.glob(str(ROOT / "oracle" / "_ref" / "_cpu_qwen*.so")), reason="oracle/_ref not built")
@pytest.mark.parametrize("ty", ALL_TYPES, ids=lambda t: t.name)
def test_qmv_bit_identical_to_reference_live(oracle_mod, ty):
    spec = importlib.util.spec_from_file_location("_cpu_qwen", glob.glob(str(ROOT / "oracle" / "_ref" / "_cpu_qwen*.so"))[0])
    ref = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(ref)
    rt = ref.CpuRuntime(tables.table("iq3s_grid"), 2)
    rng = np.random.default_rng(int(ty) + 7)
    for rows, cols, ntok in [(9, 1024, 8), (3, 256, 13), (5, 2048, 1)]:
        w = synth.baseline_rows(ty, rows, cols, rng)
        x = rng.standard_normal((ntok, cols)).astype(np.float32)
        rt.add_tensor(f"w{rows}", w.tobytes(), int(ty), cols, rows)
        rt.alloc("x", cols * ntok)
        rt.alloc("y", rows * ntok)
        rt.write("x", x.tobytes())
        rt.qmv(f"w{rows}", "x", "y", ntok)
        yr = np.frombuffer(rt.read("y"), np.float32).reshape(ntok, rows)
        assert np.array_equal(yr.view(np.uint32), oracle_mod.qmv(int(ty), w, rows, cols, x, ntok).view(np.uint32))


# ---- exact integer structure ------------------------------------------------------------------------------

@pytest.mark.parametrize("ty", QUANT_TYPES, ids=lambda t: t.name)
def test_codes_scales_reproduce_dequant_and_partials(oracle_mod, ty):
    rows, cols, ntok = 6, 512, 3
    rng = np.random.default_rng(100 + int(ty))
    w = synth.baseline_rows(ty, rows, cols, rng)
    codes, scales, mins = oracle_mod.decode_codes(int(ty), w, rows, cols)
    deq = oracle_mod.dequant_rows(int(ty), w, rows, cols)
    s = np.repeat(scales.astype(np.float64), 16, axis=1)
    m = np.repeat(mins.astype(np.float64), 16, axis=1)
    assert np.array_equal((s * codes - m).astype(np.float32), deq)  # exact product, one rounding
    x = rng.standard_normal((ntok, cols)).astype(np.float32)
    xq, _, _ = oracle_mod.quantize_x(x, ntok, cols)
    part = oracle_mod.int_partials(int(ty), w, rows, cols, xq, ntok)
    brute = np.einsum("rgk,tgk->trg", codes.reshape(rows, -1, 16).astype(np.int64), xq.reshape(ntok, -1, 16).astype(np.int64))
    assert np.array_equal(part.reshape(ntok, rows, -1), brute)


def test_quantizer_closed_form(oracle_mod):
    rng = np.random.default_rng(5)
    x = rng.standard_normal((2, 256)).astype(np.float32) * 3
    x[1, 32:64] = 0.0
    xq, xd, xs = oracle_mod.quantize_x(x, 2, 256)
    g = x.reshape(2, 8, 32)
    amax = np.abs(g).max(-1)
    assert np.array_equal(xd, (amax / np.float32(127)).astype(np.float32))
    assert np.all(np.abs(xq.astype(int)) <= 127)
    assert np.all(np.abs(xq.reshape(2, 8, 32)).max(-1)[amax > 0] == 127)
    assert np.all(xq[1, 32:64] == 0) and xd[1, 1] == 0 and xs[1, 1] == 0
    err = np.abs(xq.reshape(2, 8, 32) * xd[..., None].astype(np.float64) - g)
    assert np.all(err <= 0.5 * xd[..., None] * (1 + 1e-6) + 1e-12)
    assert np.array_equal(xs, (xd * xq.reshape(2, 8, 32).astype(np.int64).sum(-1).astype(np.float32)).astype(np.float32))


def test_argmax_semantics(oracle_mod):
    x = np.array([[1, 5, 5, 2], [np.nan, 3, np.nan, 3], [-np.inf] * 4], np.float32)
    assert oracle_mod.argmax_rows(x, 4, 3) == [1, 1, 2**31 - 1]


def test_stage_x_is_pinned_by_closed_forms(oracle_mod):
    """stage_x (the megakernel's activation staging): identities that a dropped term, a wrong sign or a
    misplaced eps would break."""
    from scipy.special import expit

    st = oracle_mod.stage_x
    rng = np.random.default_rng(61)
    x = rng.standard_normal((3, 256)) * 4.0
    x2 = rng.standard_normal((3, 256))
    nw = rng.uniform(0.5, 2.0, 256)
    assert np.array_equal(st(x, None, None, 0.0, 0), x)
    # silu(z) = z * sigmoid(z) (textbook logistic), silu(-z) = silu(z) - z, silu(0) = 0
    s = st(x, np.ones_like(x), None, 0.0, oracle_mod.STAGE_SILU_MUL)
    assert np.allclose(s, x * expit(x), rtol=1e-14, atol=1e-300)
    assert np.allclose(st(-x, np.ones_like(x), None, 0.0, oracle_mod.STAGE_SILU_MUL), s - x, rtol=1e-12, atol=1e-12)
    assert st(np.zeros((1, 32)), np.ones((1, 32)), None, 0.0, oracle_mod.STAGE_SILU_MUL).any() == False  # noqa: E712
    # the second input multiplies elementwise
    assert np.allclose(st(x, x2, None, 0.0, oracle_mod.STAGE_SILU_MUL), s * x2, rtol=1e-14, atol=1e-300)
    # NORM with unit weights and eps = 0: unit RMS per token, scale invariance, sign kept
    n = st(x, None, np.ones(256), 0.0, oracle_mod.STAGE_NORM)
    assert np.allclose(np.sqrt((n * n).mean(axis=1)), 1.0, rtol=1e-14)
    assert np.allclose(st(7.5 * x, None, np.ones(256), 0.0, oracle_mod.STAGE_NORM), n, rtol=1e-13)
    assert np.array_equal(np.sign(n), np.sign(x))
    # weights multiply after the normalisation; eps adds to the mean square: a constant row c gives
    # c / sqrt(c^2 + eps)
    assert np.allclose(st(x, None, nw, 0.0, oracle_mod.STAGE_NORM), n * nw, rtol=1e-13)
    c = st(np.full((1, 64), 3.0), None, np.ones(64), 7.0, oracle_mod.STAGE_NORM)
    assert np.allclose(c, 3.0 / 4.0, rtol=1e-15)
    # SILU_MUL is applied before NORM
    both = st(x, x2, nw, 1e-6, oracle_mod.STAGE_SILU_MUL | oracle_mod.STAGE_NORM)
    assert np.allclose(both, st(st(x, x2, None, 0.0, oracle_mod.STAGE_SILU_MUL), None, nw, 1e-6,
                                oracle_mod.STAGE_NORM), rtol=1e-14)
    # ADD does not change the staged activations
    assert np.array_equal(st(x, None, None, 0.0, oracle_mod.STAGE_ADD), x)


def test_rope_neox_is_pinned_by_rotation_properties(oracle_mod):
    """rope_neox: position 0 is the identity; each (j, j + rot/2) pair keeps its length; rotations compose
    (pos a then pos b == pos a + b per token); pair 0 turns by exactly pos radians; dims >= rot untouched."""
    r = oracle_mod.rope_neox
    rng = np.random.default_rng(62)
    heads, hd, rot = 3, 16, 10
    x = rng.standard_normal((1, heads, hd))
    assert np.allclose(r(x, heads, hd, rot, 0, 1e4), x, rtol=0, atol=0)
    y = r(x, heads, hd, rot, 7, 1e4)
    half = rot // 2
    assert np.allclose(np.hypot(y[..., :half], y[..., half:rot]), np.hypot(x[..., :half], x[..., half:rot]), rtol=1e-13)
    assert np.array_equal(y[..., rot:], x[..., rot:])
    assert np.allclose(r(r(x, heads, hd, rot, 3, 1e4), heads, hd, rot, 4, 1e4), y, rtol=1e-12, atol=1e-12)
    c, s = np.cos(7.0), np.sin(7.0)
    assert np.allclose(y[..., 0], x[..., 0] * c - x[..., half] * s, rtol=1e-14)
    # token t sits at pos0 + t
    x2 = rng.standard_normal((2, heads, hd))
    assert np.allclose(r(x2, heads, hd, rot, 5, 1e4)[1], r(x2[1:], heads, hd, rot, 6, 1e4)[0], rtol=1e-14)


def test_attention_is_pinned_by_closed_forms(oracle_mod):
    """attention: equal keys average V; one visible position returns its V row; a window of 1 returns the
    query's own position; a score gap of ln(3) weights 3:1; GQA heads read kv head h // (heads / kv_heads)."""
    at = oracle_mod.attention
    rng = np.random.default_rng(63)
    kvh, heads, hd, ms = 2, 4, 8, 12
    v = rng.standard_normal((kvh, ms, hd))
    q = rng.standard_normal((1, heads, hd))
    zero_k = np.zeros((kvh, ms, hd))
    o = at(q, zero_k, v, heads, kvh, 5)
    assert np.allclose(o[0, 0], v[0, :5].mean(0)) and np.allclose(o[0, 3], v[1, :5].mean(0))
    assert np.allclose(at(q, rng.standard_normal((kvh, ms, hd)), v, heads, kvh, 1)[0, 2], v[1, 0])
    assert np.allclose(at(q, rng.standard_normal((kvh, ms, hd)), v, heads, kvh, 7, window=1)[0, 1], v[0, 6])
    k = np.zeros((kvh, ms, hd))
    qq = np.zeros((1, heads, hd))
    qq[0, :, 0] = 1.0
    k[:, 1, 0] = np.log(3.0) * np.sqrt(hd)  # position 1 scores ln 3 above position 0
    assert np.allclose(at(qq, k, v, heads, kvh, 2)[0, 0], 0.25 * v[0, 0] + 0.75 * v[0, 1])
    # token t of a causal block sees one position more than token t - 1; bidirectional tokens all see the block
    q3 = rng.standard_normal((3, heads, hd))
    kk = rng.standard_normal((kvh, ms, hd))
    c = at(q3, kk, v, heads, kvh, 4)
    assert np.allclose(c[2], at(q3[2:], kk, v, heads, kvh, 6)[0])
    b = at(q3, kk, v, heads, kvh, 4, bidirectional=True)
    assert np.allclose(b[0], at(q3[:1], kk, v, heads, kvh, 6)[0]) and np.allclose(b[2], c[2])


def test_conv_update_is_pinned_by_closed_forms(oracle_mod):
    """conv_update: a last-tap-only filter gives silu(x_t); after K tokens the state is exactly the last K
    inputs; all-ones weights give silu(sum of the last K inputs, the old state filling the start)."""
    from scipy.special import expit

    cu = oracle_mod.conv_update
    rng = np.random.default_rng(64)
    ch, K, ntok = 5, 4, 6
    x = rng.standard_normal((ntok, ch))
    s0 = rng.standard_normal((ch, K))
    w = np.zeros((ch, K))
    w[:, -1] = 1.0
    out, st, snaps = cu(x, s0, w)
    assert np.allclose(out, x * expit(x), rtol=1e-14)
    assert np.array_equal(st, x[-K:].T) and snaps.shape == (ntok - 1, ch, K)
    assert np.array_equal(snaps[0], np.concatenate([s0[:, 1:], x[:1].T], axis=1))
    out1, _, _ = cu(x, s0, np.ones((ch, K)))
    seq = np.concatenate([s0.T, x])  # [K + ntok][ch]
    want = np.array([seq[t + 1:t + 1 + K].sum(0) for t in range(ntok)])
    assert np.allclose(out1, want * expit(want), rtol=1e-13)


def test_gated_delta_is_pinned_by_delta_rule_properties(oracle_mod):
    """gated_delta: with no decay (ssm_a = 0) and beta -> 1, writing k -> v into an empty state and reading
    with q = k returns v / sqrt(kd) (eps = 0); a second write of the same k overwrites v (delta rule, not a
    sum); beta -> 0 leaves the state decayed only; head_order picks grouped or tiled key heads."""
    gd = oracle_mod.gated_delta
    rng = np.random.default_rng(65)
    kh, vh, kd, vd = 1, 2, 8, 4
    k = rng.standard_normal(kd)
    v1, v2 = rng.standard_normal(vh * vd), rng.standard_normal(vh * vd)
    conv = np.stack([np.concatenate([k, k, v1]), np.concatenate([k, k, v2])])
    big = np.full((2, vh), 60.0)
    z = np.zeros(vh)
    out, S, snaps = gd(conv, big, np.full((2, vh), -40.0), z, z, np.zeros((vh, kd, vd)), kh, vh, kd, vd, 0.0, 0)
    assert np.allclose(out[0], v1.reshape(vh, vd) / np.sqrt(kd), rtol=1e-12)
    assert np.allclose(out[1], v2.reshape(vh, vd) / np.sqrt(kd), rtol=1e-12)
    assert np.allclose(snaps[0], np.einsum("i,hj->hij", k / np.linalg.norm(k), v1.reshape(vh, vd)), rtol=1e-12)
    s0 = rng.standard_normal((vh, kd, vd))
    ssm = np.array([-1.0, -0.5])
    _, S2, _ = gd(conv[:1], np.full((1, vh), -60.0), np.zeros((1, vh)), ssm, z, s0, kh, vh, kd, vd, 1e-6, 0)
    assert np.allclose(S2, s0 * np.exp(ssm * np.log(2.0))[:, None, None], rtol=1e-12)  # softplus(0) = ln 2
    kh2 = 2
    conv2 = rng.standard_normal((1, 2 * kh2 * kd + 4 * vd))
    o_g, _, _ = gd(conv2, big[:1, :1].repeat(4, 1), np.zeros((1, 4)), np.zeros(4), np.zeros(4), np.zeros((4, kd, vd)),
                   kh2, 4, kd, vd, 1e-6, 0)
    o_t, _, _ = gd(conv2, big[:1, :1].repeat(4, 1), np.zeros((1, 4)), np.zeros(4), np.zeros(4), np.zeros((4, kd, vd)),
                   kh2, 4, kd, vd, 1e-6, 1)
    assert np.allclose(o_g[0, 0], o_t[0, 0]) and not np.allclose(o_g[0, 1], o_t[0, 1])  # head 1: key 0 vs key 1


def test_paged_rows_round_trip():
    """oracle.paged_rows / gather_paged (KvAddr::row, qwen_runtime.cu:100-110): scattering each position's row of
    a contiguous cache through a permuted page table and gathering it back is the identity; every row lands in
    a distinct pool row, on the page the table names, at slot pos % page_size."""
    from oracle import oracle

    rng = np.random.default_rng(0)
    page, pps, kvh, hd, length = 4, 5, 3, 2, 18
    pt = rng.permutation(pps * 2)[:pps]
    pool = np.full((pps * 2, kvh, page, hd), np.nan)
    cont = rng.standard_normal((kvh, length, hd))
    flat = pool.reshape(-1, hd)
    seen = set()
    for h in range(kvh):
        rows = oracle.paged_rows(pt, page, kvh, h, np.arange(length))
        assert len(set(rows.tolist()) & seen) == 0
        seen |= set(rows.tolist())
        flat[rows] = cont[h]
        for p, r in zip(range(length), rows):
            assert r // (kvh * page) == pt[p // page] and r % page == p % page and (r // page) % kvh == h
    assert np.array_equal(oracle.gather_paged(pool, pt, page, kvh, length), cont)


def test_qgemm_f16x_is_pinned_by_brute_force_and_plain_f16(oracle_mod):
    """The fp16-activation prompt GEMM restatement: (1) pure-Python brute force on a tiny case, rounding each
    activation with struct's IEEE half packing (independent of numpy's float16); (2) for tokens whose values are
    normal fp16 numbers, bit-identical to W f16(x) with no scaling, i.e. the reference's f32_to_f16_rows_kernel
    (qwen_runtime.cu:657-661); (3) a token far outside fp16's range still gives 2^k times the in-range result."""
    rng = np.random.default_rng(3)
    rows, cols, ntok = 3, 256, 2
    for ty in (T.Q4_K, T.Q5_K):
        w = synth.baseline_rows(ty, rows, cols, rng)
        x = rng.standard_normal((ntok, cols)).astype(np.float32)
        got = oracle_mod.qgemm_f16x(int(ty), w, rows, cols, x, ntok)
        wd = oracle_mod.dequant_rows(int(ty), w, rows, cols).astype(np.float64)
        for t in range(ntok):
            m = max(abs(float(v)) for v in x[t])
            e = 0
            while 2.0 ** e <= m:
                e += 1
            while 2.0 ** (e - 1) > m:
                e -= 1
            s = 2.0 ** min(15 - e, 126)
            xb = [struct.unpack("<e", struct.pack("<e", float(v) * s))[0] for v in x[t]]
            for r in range(rows):
                want = sum(float(wd[r][k]) * xb[k] for k in range(cols)) / s
                assert abs(got[t][r] - want) <= 1e-12 * max(1.0, abs(want)), (ty, t, r)
        xn = np.where(np.abs(x) < 1e-3, np.float32(1e-3), x)  # every value a normal fp16 number
        plain = (xn.astype(np.float16).astype(np.float64) @ wd.T)
        assert np.array_equal(oracle_mod.qgemm_f16x(int(ty), w, rows, cols, xn, ntok), plain)
        big = (xn * np.float32(2.0 ** 40)).astype(np.float32)  # far above fp16's 65504
        assert np.array_equal(oracle_mod.qgemm_f16x(int(ty), w, rows, cols, big, ntok), plain * 2.0 ** 40)


def test_f16x_weights_round_q6k_once(oracle_mod):
    """f16x_weights: Q6_K's weight d f16((q - 32) sc) lies within 2^-11 of the exact dequantized weight (a wrong
    scale or element mapping would be off by far more), equals it wherever |(q - 32) sc| <= 2048 (exact in fp16),
    and matches a per-element struct-rounded restatement; every other type is exact."""
    rng = np.random.default_rng(9)
    rows, cols = 5, 512
    raw = synth.baseline_rows(T.Q6_K, rows, cols, rng)
    ex = oracle_mod.dequant_rows(int(T.Q6_K), raw, rows, cols).astype(np.float64)
    w = oracle_mod.f16x_weights(int(T.Q6_K), raw, rows, cols)
    assert np.all(np.abs(w - ex) <= 2.0 ** -11 * np.abs(ex))
    codes, _, _ = oracle_mod.decode_codes(int(T.Q6_K), raw, rows, cols)
    blk = np.frombuffer(bytes(raw), np.uint8)[: rows * (cols // 256) * 210].reshape(rows, cols // 256, 210)
    for r in range(rows):
        for e in range(cols):
            b, j = divmod(e, 256)
            sc = int(np.int8(blk[r, b, 192 + j // 16]))
            d = struct.unpack("<e", bytes(blk[r, b, 208:210]))[0]
            prod = int(codes[r, e]) * sc
            want = struct.unpack("<e", struct.pack("<e", float(prod)))[0] * d
            assert w[r, e] == want, (r, e)
            if abs(prod) <= 2048:
                assert w[r, e] == ex[r, e]
    assert (w != ex).any()  # the shape exercises the rounding
    raw4 = synth.baseline_rows(T.Q4_K, rows, cols, rng)
    assert np.array_equal(oracle_mod.f16x_weights(int(T.Q4_K), raw4, rows, cols),
                          oracle_mod.dequant_rows(int(T.Q4_K), raw4, rows, cols).astype(np.float64))
