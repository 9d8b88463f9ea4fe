"""Sequence ops on the GPU through the runtime: the multi-sequence (_seg) forms over paged KV caches and per-slot
recurrent state, the verification-pass controls (write_state), fp16 SSM state, and the qwen35 shapes.

References: Runtime_set_paging / set_segments and the *_seg ops (qwen_runtime.cu:2333-2565), conv_update_kernel
and gated_delta_reg_kernel (qwen_runtime.cu:397-512), concat_rows / zero_range (qwen_runtime.cu:2567-2600).
Expected values come from the float64 restatements in oracle/oracle.py, applied per segment to the slot's
cache gathered out of the page pool (oracle.gather_paged, pinned in test_oracle.py).
"""
from __future__ import annotations

import numpy as np
import pytest

from vinf_3080ti_amd import GGUFTensorType as T

pytestmark = pytest.mark.gpu

# qwen35-27B gated-delta and attention shapes
QW_KH, QW_VH, QW_KD, QW_VD, QW_K = 16, 48, 128, 128, 4
QW_HEADS, QW_KVH, QW_HD = 24, 4, 256


@pytest.fixture(scope="module")
def rt():
    torch = pytest.importorskip("torch")
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    from vinf_3080ti_amd.runtime import HipWeightRuntime

    return HipWeightRuntime()


def put(rt, name: str, a, elem: int = 4) -> None:
    a = np.ascontiguousarray(a, np.float32 if elem == 4 else np.float16).reshape(-1)
    rt.alloc(name, a.size, elem)
    rt.write(name, a.tobytes())


def get(rt, name: str, shape) -> np.ndarray:
    return np.array(rt.read_floats(name), np.float64).reshape(shape)


def put_weight(rt, name: str, a) -> None:
    a = np.ascontiguousarray(a, np.float32).reshape(-1)
    rt.upload_raw(name, a.tobytes(), T.F32, a.size, 1)


def gd_inputs(rng, ntok, kh, vh, kd, vd):
    cdim = 2 * kh * kd + vh * vd
    return dict(conv=rng.standard_normal((ntok, cdim)).astype(np.float32),
                b=rng.standard_normal((ntok, vh)).astype(np.float32),
                a=rng.standard_normal((ntok, vh)).astype(np.float32),
                ssm_a=-rng.uniform(0.1, 2.0, vh).astype(np.float32),
                dt=rng.standard_normal(vh).astype(np.float32))


GD_TOL = dict(rtol=1e-4, atol=2e-5)


@pytest.mark.parametrize("kh,vh,kd,vd,ntok", [(QW_KH, QW_VH, QW_KD, QW_VD, 1), (QW_KH, QW_VH, QW_KD, QW_VD, 8),
                                              (2, 6, 256, 64, 3), (1, 3, 40, 100, 2), (4, 4, 32, 8, 5),
                                              (2, 4, 24, 10, 3), (1, 2, 66, 36, 2), (2, 4, 64, 32, 37),
                                              (QW_KH, QW_VH, QW_KD, QW_VD, 20)])
def test_gated_delta_shapes(rt, oracle_mod, kh, vh, kd, vd, ntok):
    """The register-resident gated delta at the qwen35 shape (decode and an 8-row verify pass), kd 256, and
    ragged kd / vd (rows and columns past the state's edge masked): outputs, state and snapshots. vd and kd
    multiples of 4 take the column-quad kernel (20 and 37 rows: its 16-token input chunks, the last one partial);
    vd 10 and kd 66 the one-column kernel."""
    rng = np.random.default_rng(kd * vd + ntok)
    inp = gd_inputs(rng, ntok, kh, vh, kd, vd)
    s0 = (rng.standard_normal((vh, kd, vd)) * 0.1).astype(np.float32)
    put_weight(rt, "gsa", inp["ssm_a"])
    put_weight(rt, "gdt", inp["dt"])
    for name in ("conv", "b", "a"):
        put(rt, "g" + name, inp[name])
    put(rt, "gs", s0)
    put(rt, "go", np.zeros(ntok * vh * vd))
    put(rt, "gsn", np.zeros(max(ntok - 1, 1) * vh * kd * vd))
    rt.gated_delta("gconv", "gb", "ga", "gsa", "gdt", "gs", "go", kh, vh, kd, vd, 1e-6, 0, ntok,
                   "gsn" if ntok > 1 else None)
    out, S, snaps = oracle_mod.gated_delta(inp["conv"], inp["b"], inp["a"], inp["ssm_a"], inp["dt"], s0, kh, vh, kd,
                                           vd, 1e-6, 0)
    assert np.allclose(get(rt, "go", (ntok, vh, vd)), out, **GD_TOL)
    assert np.allclose(get(rt, "gs", (vh, kd, vd)), S, **GD_TOL)
    if ntok > 1:
        assert np.allclose(get(rt, "gsn", (-1, vh, kd, vd))[:ntok - 1], snaps, **GD_TOL)
    # write_state = 0: same outputs, state untouched (a verification pass)
    put(rt, "gs", s0)
    rt.gated_delta("gconv", "gb", "ga", "gsa", "gdt", "gs", "go", kh, vh, kd, vd, 1e-6, 0, ntok, None, 0)
    assert np.allclose(get(rt, "go", (ntok, vh, vd)), out, **GD_TOL)
    assert np.array_equal(np.array(rt.read_floats("gs"), np.float32), s0.reshape(-1))
    for n in ("gsa", "gdt"):
        rt.free(n)


def test_conv_update_write_state_zero(rt, oracle_mod):
    """conv_update with write_state = 0 (qwen_runtime.cu:402,421-422): outputs and snapshots as usual, the state
    unchanged; K = 4 at the qwen35 conv width (10240 channels)."""
    rng = np.random.default_rng(5)
    ch, K, ntok = 10240, QW_K, 4
    x = rng.standard_normal((ntok, ch)).astype(np.float32)
    s0 = rng.standard_normal((ch, K)).astype(np.float32)
    w = (rng.standard_normal((ch, K)) * 0.5).astype(np.float32)
    rt.upload_raw("cw", w.tobytes(), T.F32, K, ch)
    put(rt, "cx", x)
    put(rt, "cs", s0)
    put(rt, "co", np.zeros((ntok, ch)))
    put(rt, "csn", np.zeros((ntok - 1, ch, K)))
    rt.conv_update("cx", "cs", "cw", "co", ch, K, ntok, "csn", 0)
    out, _, snaps = oracle_mod.conv_update(x, s0, w)
    assert np.allclose(get(rt, "co", (ntok, ch)), out, rtol=1e-5, atol=1e-6)
    assert np.array_equal(get(rt, "csn", (ntok - 1, ch, K)), snaps)
    assert np.array_equal(np.array(rt.read_floats("cs"), np.float32), s0.reshape(-1))
    rt.free("cw")


@pytest.mark.parametrize("K", [1, 3, 8])
def test_conv_update_kernel_sizes(rt, oracle_mod, K):
    rng = np.random.default_rng(K)
    ch, ntok = 77, 3
    x = rng.standard_normal((ntok, ch)).astype(np.float32)
    s0 = rng.standard_normal((ch, K)).astype(np.float32)
    w = rng.standard_normal((ch, K)).astype(np.float32)
    rt.upload_raw("cw", w.tobytes(), T.F32, K, ch)
    put(rt, "cx", x)
    put(rt, "cs", s0)
    put(rt, "co", np.zeros((ntok, ch)))
    rt.conv_update("cx", "cs", "cw", "co", ch, K, ntok)
    out, st, _ = oracle_mod.conv_update(x, s0, w)
    assert np.allclose(get(rt, "co", (ntok, ch)), out, rtol=1e-5, atol=1e-6)
    assert np.array_equal(get(rt, "cs", (ch, K)), st)
    rt.free("cw")
    with pytest.raises(ValueError):
        rt.conv_update("cx", "cs", "cw", "co", ch, 9, ntok)


@pytest.mark.parametrize("elem", [4, 2])
@pytest.mark.parametrize("ntok,seq_len,bidirectional,window", [(1, 700, 0, 0), (5, 33, 0, 0), (3, 90, 1, 0),
                                                               (2, 400, 0, 128)])
def test_attention_head_dim_256(rt, oracle_mod, elem, ntok, seq_len, bidirectional, window):
    """attention at the qwen35 full-attention shape: 24 heads over 4 kv heads, hd 256 (all four accumulator
    slots and the largest LDS arrays of the kernel), fp32 and fp16 caches, causal / bidirectional / window."""
    rng = np.random.default_rng(seq_len + 10 * ntok + elem)
    heads, kvh, hd, max_seq = QW_HEADS, QW_KVH, QW_HD, 720
    q = rng.standard_normal((ntok, heads, hd)).astype(np.float32)
    dt = np.float32 if elem == 4 else np.float16
    kc = (rng.standard_normal((kvh, max_seq, hd)) * 0.2).astype(dt)
    vc = rng.standard_normal((kvh, max_seq, hd)).astype(dt)
    put(rt, "aq", q)
    put(rt, "ao", np.zeros(q.size))
    put(rt, "akc", kc, elem)
    put(rt, "avc", vc, elem)
    rt.attention("aq", "akc", "avc", "ao", heads, kvh, hd, max_seq, seq_len, ntok, bidirectional, window)
    ref = oracle_mod.attention(q, kc, vc, heads, kvh, seq_len, bool(bidirectional), window)
    assert np.allclose(get(rt, "ao", (ntok, heads, hd)), ref, rtol=2e-5, atol=2e-5)


def test_concat_rows_and_zero_range(rt):
    rng = np.random.default_rng(9)
    rows, width = 7, 1000
    a = rng.standard_normal((rows, width)).astype(np.float32)
    b = rng.standard_normal((rows, width)).astype(np.float32)
    put(rt, "ca", a)
    put(rt, "cb", b)
    put(rt, "cd", np.full(2 * rows * width, 5.0))
    rt.concat_rows("cd", "ca", "cb", rows, width)
    assert np.array_equal(np.array(rt.read_floats("cd"), np.float32).reshape(rows, 2 * width),
                          np.concatenate([a, b], axis=1))
    rt.zero_range("cd", 3, 1001)
    got = np.array(rt.read_floats("cd"), np.float32)
    want = np.concatenate([a, b], axis=1).reshape(-1)
    want[3:1004] = 0
    assert np.array_equal(got, want)
    put(rt, "ch", np.arange(11), 2)
    rt.zero_range("ch", 1, 5)  # fp16 buffer: odd element offset and count
    assert rt.read_floats("ch") == [0, 0, 0, 0, 0, 0, 6, 7, 8, 9, 10]
    with pytest.raises(ValueError):
        rt.zero_range("cd", 2 * rows * width - 3, 4)
    with pytest.raises(ValueError):
        rt.concat_rows("cd", "ca", "cb", rows + 1, width)


# ---- multi-sequence passes ----------------------------------------------------------------------------------

PAGE, PPS, SLOTS = 16, 12, 5  # 192 positions per sequence


def paging(rt, rng, kvh, hd, elem):
    """A page pool shared by SLOTS sequences, pages handed out in a random order."""
    npages = PPS * SLOTS
    pt = rng.permutation(npages).astype(np.int32).reshape(SLOTS, PPS)
    rt.alloc("pt", pt.size)
    rt.write("pt", pt.tobytes())
    rt.set_paging("pt", PAGE, PPS, SLOTS)
    dt = np.float32 if elem == 4 else np.float16
    pool_k = (rng.standard_normal((npages, kvh, PAGE, hd)) * 0.3).astype(dt)
    pool_v = rng.standard_normal((npages, kvh, PAGE, hd)).astype(dt)
    put(rt, "pk", pool_k, elem)
    put(rt, "pv", pool_v, elem)
    return pt, pool_k, pool_v


def test_set_segments_contract(rt):
    from vinf_3080ti_amd.runtime import Runtime

    fresh = Runtime()
    with pytest.raises(RuntimeError):
        fresh.set_segments([(0, 0, 1)])
    fresh.alloc("pt", PPS * SLOTS)
    fresh.set_paging("pt", PAGE, PPS, SLOTS)
    with pytest.raises(RuntimeError):
        fresh.rope_seg("pt", 1, 4, 4, 1e4)
    assert fresh.set_segments([(0, 5, 3), (2, 0, 4)]) == 7
    assert fresh.set_segments([(0, 5, 3, 10), (1, 0, 2)]) == 15  # explicit row0 places later rows too
    for bad in ([(SLOTS, 0, 1)], [(0, PAGE * PPS - 1, 2)], [(0, 0, 0)], [(-1, 0, 1)], []):
        with pytest.raises(ValueError):
            fresh.set_segments(bad)
    with pytest.raises(ValueError):
        fresh.set_paging("pt", 0, PPS, SLOTS)


@pytest.mark.parametrize("elem", [4, 2])
def test_rope_kv_append_attention_seg(rt, oracle_mod, elem):
    """A decode + verify pass over three sequences (1, 4 and 3 rows at different positions, one segment placed
    by an explicit row0 past a gap): rope_seg, kv_append_seg into random pages, attention_seg over each
    sequence's own pages; pages of other slots are untouched."""
    rng = np.random.default_rng(40 + elem)
    heads, kvh, hd, rot, base = 8, 2, 64, 32, 1e6
    pt, pool_k, pool_v = paging(rt, rng, kvh, hd, elem)
    segs = [(3, 150, 1), (0, 17, 4), (4, 60, 3, 7)]
    nrows = rt.set_segments(segs)
    assert nrows == 10
    q = rng.standard_normal((nrows, heads, hd)).astype(np.float32)
    k = rng.standard_normal((nrows, kvh, hd)).astype(np.float32)
    v = rng.standard_normal((nrows, kvh, hd)).astype(np.float32)
    put(rt, "sq", q)
    put(rt, "sk", k)
    put(rt, "sv", v)
    put(rt, "so", np.zeros(q.size))
    rt.rope_seg("sq", heads, hd, rot, base)
    rt.rope_seg("sk", kvh, hd, rot, base)
    rt.kv_append_seg("sk", "sv", "pk", "pv", kvh, hd)
    rt.attention_seg("sq", "pk", "pv", "so", heads, kvh, hd)
    got_q = get(rt, "sq", (nrows, heads, hd))
    got_k = get(rt, "sk", (nrows, kvh, hd))
    got_o = get(rt, "so", (nrows, heads, hd))
    dt = np.float32 if elem == 4 else np.float16
    pk_got = np.array(rt.read_floats("pk"), np.float32).reshape(pool_k.shape).astype(dt)
    pv_got = np.array(rt.read_floats("pv"), np.float32).reshape(pool_v.shape).astype(dt)
    exp_k, exp_v = pool_k.copy(), pool_v.copy()
    fk, fv = exp_k.reshape(-1, hd), exp_v.reshape(-1, hd)
    rowmap = [(slot, pos0, n, r0) for (slot, pos0, n, *r) in segs for r0 in [r[0] if r else None]]
    row = 0
    placed = []
    for slot, pos0, n, r0 in rowmap:
        row = r0 if r0 is not None else row
        placed.append((slot, pos0, n, row))
        rq = oracle_mod.rope_neox(q[row:row + n], heads, hd, rot, pos0, base)
        rk = oracle_mod.rope_neox(k[row:row + n], kvh, hd, rot, pos0, base)
        assert np.allclose(got_q[row:row + n], rq, rtol=1e-5, atol=2e-6)
        assert np.allclose(got_k[row:row + n], rk, rtol=1e-5, atol=2e-6)
        for h in range(kvh):
            idx = oracle_mod.paged_rows(pt[slot], PAGE, kvh, h, np.arange(pos0, pos0 + n))
            fk[idx] = got_k[row:row + n, h].astype(np.float32).astype(dt)
            fv[idx] = v[row:row + n, h].astype(dt)
        row += n
    assert np.array_equal(pk_got, exp_k)
    assert np.array_equal(pv_got, exp_v)
    for slot, pos0, n, row in placed:
        kc = oracle_mod.gather_paged(exp_k, pt[slot], PAGE, kvh, pos0 + n)
        vc = oracle_mod.gather_paged(exp_v, pt[slot], PAGE, kvh, pos0 + n)
        ref = oracle_mod.attention(got_q[row:row + n].astype(np.float32), kc, vc, heads, kvh, pos0 + 1)
        assert np.allclose(got_o[row:row + n], ref, rtol=2e-5, atol=2e-5), (slot, pos0, n)
    with pytest.raises(ValueError):
        rt.attention_seg("sq", "pk", "pv", "so", heads, 3, hd)


@pytest.mark.parametrize("state_elem", [4, 2])
def test_conv_and_gated_delta_seg(rt, oracle_mod, state_elem):
    """conv_update_seg and gated_delta_seg over three slots of the per-slot state (qwen35 head shape, 2 value
    heads' worth of key heads kept small): each segment steps its own slot; other slots untouched; fp16 state
    is rounded once at the end of the pass; write_state = 0 leaves every slot as it was."""
    rng = np.random.default_rng(70 + state_elem)
    kh, vh, kd, vd, K, slots = 2, 6, QW_KD, QW_VD, QW_K, 4
    rt.alloc("pt", PPS * SLOTS)
    rt.set_paging("pt", PAGE, PPS, slots)
    segs = [(2, 30, 3), (0, 0, 1), (3, 9, 2)]
    n = rt.set_segments(segs)
    inp = gd_inputs(rng, n, kh, vh, kd, vd)
    cdim = inp["conv"].shape[1]
    x = rng.standard_normal((n, cdim)).astype(np.float32)
    w = (rng.standard_normal((cdim, K)) * 0.5).astype(np.float32)
    cs0 = rng.standard_normal((slots, cdim, K)).astype(np.float32)
    sdt = np.float32 if state_elem == 4 else np.float16
    s0 = (rng.standard_normal((slots, vh, kd, vd)) * 0.1).astype(sdt)
    rt.upload_raw("cw", w.tobytes(), T.F32, K, cdim)
    put_weight(rt, "gsa", inp["ssm_a"])
    put_weight(rt, "gdt", inp["dt"])
    put(rt, "cx", x)
    put(rt, "ccs", cs0)
    put(rt, "cconv", np.zeros((n, cdim)))
    put(rt, "gb", inp["b"])
    put(rt, "ga", inp["a"])
    put(rt, "gs", s0, state_elem)
    put(rt, "go", np.zeros(n * vh * vd))
    for write in (0, 1):
        rt.conv_update_seg("cx", "ccs", "cw", "cconv", cdim, K, None, write)
        rt.gated_delta_seg("cconv", "gb", "ga", "gsa", "gdt", "gs", "go", kh, vh, kd, vd, 1e-6, 1, None, write)
        conv_out = get(rt, "cconv", (n, cdim))
        out = get(rt, "go", (n, vh, vd))
        cs = get(rt, "ccs", (slots, cdim, K))
        st = np.array(rt.read_floats("gs"), np.float64).reshape(slots, vh, kd, vd)
        row = 0
        for slot, _, m in segs:
            co, cst, _ = oracle_mod.conv_update(x[row:row + m], cs0[slot], w)
            assert np.allclose(conv_out[row:row + m], co, rtol=1e-5, atol=1e-6)
            o, S, _ = oracle_mod.gated_delta(conv_out[row:row + m].astype(np.float32), inp["b"][row:row + m],
                                             inp["a"][row:row + m], inp["ssm_a"], inp["dt"],
                                             s0[slot].astype(np.float32), kh, vh, kd, vd, 1e-6, 1)
            assert np.allclose(out[row:row + m], o, **GD_TOL), slot
            if write:
                assert np.array_equal(cs[slot], cst), slot
                assert np.allclose(st[slot], S.astype(sdt).astype(np.float64), rtol=1e-3 if state_elem == 2 else 1e-4,
                                   atol=2e-5), slot
            row += m
        untouched = [1] if write else range(slots)
        for slot in untouched:
            assert np.array_equal(cs[slot], cs0[slot])
            assert np.array_equal(st[slot], s0[slot].astype(np.float64))
    if state_elem == 2:
        put(rt, "gsn", np.zeros(n * vh * kd * vd))
        rt.set_segments([(0, 0, 2)])
        with pytest.raises(ValueError):
            rt.gated_delta_seg("cconv", "gb", "ga", "gsa", "gdt", "gs", "go", kh, vh, kd, vd, 1e-6, 1, "gsn")
    rt.set_segments(segs)
    put(rt, "csn", np.zeros(n * cdim * K))
    with pytest.raises(ValueError):  # snapshots need a single-segment pass
        rt.conv_update_seg("cx", "ccs", "cw", "cconv", cdim, K, "csn")
    for name in ("cw", "gsa", "gdt"):
        rt.free(name)


def test_gated_delta_seg_snapshots_single_segment(rt, oracle_mod):
    """A verification pass of one sequence: snapshots after each row but the last, state untouched; then the
    commit replay of the kept rows (explicit row0) advances the slot to the snapshot of the last kept row."""
    rng = np.random.default_rng(77)
    kh, vh, kd, vd, slots, n = 1, 2, 64, 64, 3, 5
    rt.alloc("pt", PPS * SLOTS)
    rt.set_paging("pt", PAGE, PPS, slots)
    inp = gd_inputs(rng, n, kh, vh, kd, vd)
    s0 = (rng.standard_normal((slots, vh, kd, vd)) * 0.1).astype(np.float32)
    put_weight(rt, "gsa", inp["ssm_a"])
    put_weight(rt, "gdt", inp["dt"])
    for name in ("conv", "b", "a"):
        put(rt, "g" + name, inp[name])
    put(rt, "gs", s0)
    put(rt, "go", np.zeros(n * vh * vd))
    put(rt, "gsn", np.zeros((n - 1) * vh * kd * vd))
    rt.set_segments([(1, 40, n)])
    rt.gated_delta_seg("gconv", "gb", "ga", "gsa", "gdt", "gs", "go", kh, vh, kd, vd, 1e-6, 0, "gsn", 0)
    _, _, snaps = oracle_mod.gated_delta(inp["conv"], inp["b"], inp["a"], inp["ssm_a"], inp["dt"], s0[1], kh, vh, kd,
                                         vd, 1e-6, 0)
    assert np.allclose(get(rt, "gsn", (n - 1, vh, kd, vd)), snaps, **GD_TOL)
    assert np.array_equal(np.array(rt.read_floats("gs"), np.float32), s0.reshape(-1))
    keep = 3
    rt.set_segments([(1, 40, keep, 0)])
    rt.gated_delta_seg("gconv", "gb", "ga", "gsa", "gdt", "gs", "go", kh, vh, kd, vd, 1e-6, 0)
    st = get(rt, "gs", (slots, vh, kd, vd))
    assert np.allclose(st[1], snaps[keep - 1], **GD_TOL)
    assert np.array_equal(st[0], s0[0]) and np.array_equal(st[2], s0[2])
    rt.free("gsa")
    rt.free("gdt")


# ---- prompt passes: the tiled MFMA attention (more than VQ_ATTN_ROW_MAX rows) -------------------------------

@pytest.mark.parametrize("elem", [4, 2])
@pytest.mark.parametrize("heads,kvh,hd", [(QW_HEADS, QW_KVH, QW_HD), (8, 2, 128), (6, 6, 64), (4, 1, 40)])
@pytest.mark.parametrize("ntok,seq_len,bidirectional,window", [(37, 1, 0, 0), (16, 300, 0, 0), (9, 50, 1, 0),
                                                               (70, 20, 0, 33)])
@pytest.mark.parametrize("qmag", [1.0, 1e-36])
def test_prompt_attention_matches_oracle(rt, oracle_mod, elem, heads, kvh, hd, ntok, seq_len, bidirectional, window,
                                         qmag):
    """attention over more than 8 query rows (the MFMA kernel; the reference's tiled / tensor-core prompt kernels,
    qwen_runtime.cu:181-393): GQA groups of 6, 4, 1 and 4 heads (one workgroup holds 4), hd 256 / 128 / 64 and a
    ragged 40, causal from position 0, after a cached prefix, bidirectional and sliding window; fp32 operands
    and accumulation, so held to the decode kernel's bar."""
    rng = np.random.default_rng(ntok * 31 + hd + heads + elem + window)
    max_seq = seq_len + ntok + 3
    q = (rng.standard_normal((ntok, heads, hd)) * qmag).astype(np.float32)
    dt = np.float32 if elem == 4 else np.float16
    kc = (rng.standard_normal((kvh, max_seq, hd)) * 0.3).astype(dt)
    vc = rng.standard_normal((kvh, max_seq, hd)).astype(dt)
    put(rt, "aq", q)
    put(rt, "ao", np.full(q.size, np.nan))
    put(rt, "akc", kc, elem)
    put(rt, "avc", vc, elem)
    rt.attention("aq", "akc", "avc", "ao", heads, kvh, hd, max_seq, seq_len, ntok, bidirectional, window)
    ref = oracle_mod.attention(q, kc, vc, heads, kvh, seq_len, bool(bidirectional), window)
    assert np.allclose(get(rt, "ao", (ntok, heads, hd)), ref, rtol=2e-5, atol=2e-5)


@pytest.mark.parametrize("elem", [4, 2])
def test_prompt_attention_seg(rt, oracle_mod, elem):
    """attention_seg of a mixed pass: a 45-row prompt segment, an 11-row one after a cached prefix and two decode
    rows, over paged caches (the MFMA kernel takes the whole pass)."""
    rng = np.random.default_rng(123 + elem)
    heads, kvh, hd = QW_HEADS, QW_KVH, QW_HD
    pt, pool_k, pool_v = paging(rt, rng, kvh, hd, elem)
    segs = [(1, 0, 45), (4, 100, 11), (2, 150, 1), (0, 7, 1)]
    n = rt.set_segments(segs)
    q = rng.standard_normal((n, heads, hd)).astype(np.float32)
    put(rt, "sq", q)
    put(rt, "so", np.full(q.size, np.nan))
    rt.attention_seg("sq", "pk", "pv", "so", heads, kvh, hd)
    got = get(rt, "so", (n, heads, hd))
    row = 0
    for slot, pos0, m in segs:
        kc = oracle_mod.gather_paged(pool_k, pt[slot], PAGE, kvh, pos0 + m)
        vc = oracle_mod.gather_paged(pool_v, pt[slot], PAGE, kvh, pos0 + m)
        ref = oracle_mod.attention(q[row:row + m], kc, vc, heads, kvh, pos0 + 1)
        assert np.allclose(got[row:row + m], ref, rtol=2e-5, atol=2e-5), (slot, pos0, m)
        row += m


@pytest.mark.parametrize("elem", [4, 2])
@pytest.mark.parametrize("ntok,seq_len,window", [(1, 4096, 0), (8, 1000, 0), (3, 2, 0), (5, 700, 100)])
def test_decode_attention_split_and_per_row_kernels(oracle_mod, elem, ntok, seq_len, window):
    """Both decode kernels through the C ABI on the same inputs: vq_attention (one workgroup per head and row) and
    vq_attention_ws (the context split over ~512 workgroups on fp32 MFMA, chunks merged in order), at the qwen35
    head shape, against the float64 restatement; the split kernel is bit-identical on a rerun."""
    torch = pytest.importorskip("torch")
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    from vinf_3080ti_amd import _lib

    lib = _lib.load()
    assert lib.vq_init() == 0
    rng = np.random.default_rng(seq_len + ntok + elem)
    heads, kvh, hd = QW_HEADS, QW_KVH, QW_HD
    max_seq = seq_len + ntok + 5
    dt = np.float32 if elem == 4 else np.float16
    q = rng.standard_normal((ntok, heads, hd)).astype(np.float32)
    kc = (rng.standard_normal((kvh, max_seq, hd)) * 0.3).astype(dt)
    vc = rng.standard_normal((kvh, max_seq, hd)).astype(dt)
    qd, kd_, vd_ = (torch.from_numpy(a).cuda() for a in (q, kc, vc))
    nws = lib.vq_attention_workspace_bytes(heads, kvh, hd, seq_len, ntok, window)
    assert nws > 0
    ws = torch.empty(nws, dtype=torch.uint8, device="cuda")
    outs = []
    for use_ws in (False, True, True):
        o = torch.full_like(qd, float("nan"))
        if use_ws:
            st = lib.vq_attention_ws(qd.data_ptr(), kd_.data_ptr(), vd_.data_ptr(), o.data_ptr(), elem, heads, kvh, hd,
                                     max_seq, seq_len, ntok, 0, window, ws.data_ptr(), nws, None)
        else:
            st = lib.vq_attention(qd.data_ptr(), kd_.data_ptr(), vd_.data_ptr(), o.data_ptr(), elem, heads, kvh, hd,
                                  max_seq, seq_len, ntok, 0, window, None)
        assert st == 0, lib.vq_status_string(st)
        torch.cuda.synchronize()
        outs.append(o.cpu().numpy())
    ref = oracle_mod.attention(q, kc, vc, heads, kvh, seq_len, False, window)
    for got in outs:
        assert np.allclose(got, ref, rtol=2e-5, atol=2e-5)
    assert np.array_equal(outs[1].view(np.uint32), outs[2].view(np.uint32))
    assert lib.vq_attention_ws(qd.data_ptr(), kd_.data_ptr(), vd_.data_ptr(), qd.data_ptr(), elem, heads, kvh, hd,
                               max_seq, seq_len, ntok, 0, window, ws.data_ptr(), nws - 300, None) == _lib.VQ_ERR_WORKSPACE


@pytest.mark.parametrize("heads,kvh,hd,ntok,seq_len,qmag", [(32, 2, 128, 8, 2000, 1.0), (8, 8, 64, 1, 5000, 1.0),
                                                            (24, 4, 256, 1, 33, 1e3), (24, 4, 256, 3, 300, 1e-3),
                                                            (4, 1, 128, 7, 129, 1.0), (24, 4, 256, 8, 9000, 1.0),
                                                            (24, 4, 256, 2, 300, 1e-36), (8, 2, 128, 1, 700, 0.0)])
def test_decode_attention_fp16_cache_shapes(oracle_mod, heads, kvh, hd, ntok, seq_len, qmag):
    """The fp16-cache decode kernel (f16 MFMA on exact hi/lo splits of the query and the softmax weights) over
    head shapes 64/128/256, groups of 1 to 16 query heads per kv head (up to 8 query groups of 16 vectors), one
    chunk (no merge) and many, and queries of magnitude 1e3, 1e-3, 1e-36 and 0 (the per-vector power-of-two
    scaling, capped so that tiny queries give near-uniform weights, not NaN): within the fp32 bar of the float64
    restatement, bit-identical on a rerun."""
    torch = pytest.importorskip("torch")
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    from vinf_3080ti_amd import _lib

    lib = _lib.load()
    assert lib.vq_init() == 0
    rng = np.random.default_rng(heads * hd + ntok + seq_len)
    max_seq = seq_len + ntok + 3
    q = (rng.standard_normal((ntok, heads, hd)) * qmag).astype(np.float32)
    kc = (rng.standard_normal((kvh, max_seq, hd)) * 0.3 / max(qmag, 1.0) ** 0.5).astype(np.float16)
    vc = rng.standard_normal((kvh, max_seq, hd)).astype(np.float16)
    qd, kd_, vd_ = (torch.from_numpy(a).cuda() for a in (q, kc, vc))
    nws = lib.vq_attention_workspace_bytes(heads, kvh, hd, seq_len, ntok, 0)
    ws = torch.empty(nws, dtype=torch.uint8, device="cuda")
    outs = []
    for _ in range(2):
        o = torch.full_like(qd, float("nan"))
        st = lib.vq_attention_ws(qd.data_ptr(), kd_.data_ptr(), vd_.data_ptr(), o.data_ptr(), 2, heads, kvh, hd,
                                 max_seq, seq_len, ntok, 0, 0, ws.data_ptr(), nws, None)
        assert st == 0, lib.vq_status_string(st)
        torch.cuda.synchronize()
        outs.append(o.cpu().numpy())
    ref = oracle_mod.attention(q, kc, vc, heads, kvh, seq_len, False, 0)
    assert np.allclose(outs[0], ref, rtol=2e-5, atol=2e-5), float(np.abs(outs[0] - ref).max())
    assert np.array_equal(outs[0].view(np.uint32), outs[1].view(np.uint32))


@pytest.mark.parametrize("elem", [2, 4])
def test_decode_attention_seg_paged_head_dim_256(rt, oracle_mod, elem):
    """Decode and verify rows of three sequences over paged caches at the qwen35 head shape (24 heads over 4 kv
    heads, hd 256): the split kernel (f16 MFMA for the fp16 pool) with the page table read per key block."""
    rng = np.random.default_rng(77 + elem)
    heads, kvh, hd = QW_HEADS, QW_KVH, QW_HD
    pt, pool_k, pool_v = paging(rt, rng, kvh, hd, elem)
    segs = [(0, 150, 1), (2, 120, 4), (1, 17, 3)]
    n = rt.set_segments(segs)
    q = rng.standard_normal((n, heads, hd)).astype(np.float32)
    put(rt, "sq", q)
    put(rt, "so", np.full(q.size, np.nan))
    rt.attention_seg("sq", "pk", "pv", "so", heads, kvh, hd)
    got = get(rt, "so", (n, heads, hd))
    row = 0
    for slot, pos0, m in segs:
        kc = oracle_mod.gather_paged(pool_k, pt[slot], PAGE, kvh, pos0 + m)
        vc = oracle_mod.gather_paged(pool_v, pt[slot], PAGE, kvh, pos0 + m)
        ref = oracle_mod.attention(q[row:row + m], kc, vc, heads, kvh, pos0 + 1)
        assert np.allclose(got[row:row + m], ref, rtol=2e-5, atol=2e-5), (slot, pos0, m)
        row += m
