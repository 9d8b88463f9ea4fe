"""The C-ABI library loads, exports every symbol include/vq.h declares, and rejects bad arguments on the
host before anything reaches the GPU; the Python runtime's validation mirrors the reference's. CPU only."""
from __future__ import annotations

import ctypes
import re

import pytest

from conftest import ROOT
from vinf_3080ti_amd import _lib, gguf_types, runtime
from vinf_3080ti_amd import GGUFTensorType as T
from vinf_3080ti_amd.build import LIB

HEADER = ROOT / "include" / "vq.h"


def declared_symbols() -> list[str]:
    text = re.sub(r"/\*.*?\*/", "", HEADER.read_text(), flags=re.S)
    return sorted(set(re.findall(r"\b(vq_\w+)\s*\(", text)))


@pytest.fixture(scope="module")
def lib():
    if not LIB.exists():
        pytest.fail(f"{LIB} is not built (run __graft_entry__.build())")
    return _lib.load()


def test_header_and_binding_agree():
    assert declared_symbols() == sorted(_lib.SIGNATURES)


def test_library_exports_every_declared_symbol(lib):
    raw = ctypes.CDLL(str(LIB))
    for name in declared_symbols():
        assert hasattr(raw, name), name


def test_traits_match_python_table(lib):
    for ty, (bs, ts) in gguf_types.TYPE_TRAITS.items():
        b, t = ctypes.c_int(), ctypes.c_int()
        assert lib.vq_type_traits(int(ty), ctypes.byref(b), ctypes.byref(t)) == 0
        assert (b.value, t.value) == (bs, ts)
        assert lib.vq_row_bytes(int(ty), 5120 if bs <= 256 and 5120 % bs == 0 else bs) == (5120 // bs * ts if 5120 % bs == 0 else ts)
    assert lib.vq_type_traits(2, None, None) == _lib.VQ_ERR_TYPE  # Q4_0 has no matvec here
    assert lib.vq_row_bytes(int(T.Q4_K), 100) == -1


def test_host_side_argument_checks(lib):
    fake = ctypes.c_void_p(0x1000)  # never dereferenced: every call below fails its host-side checks
    assert lib.vq_qmv(2, fake, 4, 256, fake, 1, fake, fake, 1 << 20, None) == _lib.VQ_ERR_TYPE
    assert lib.vq_qmv(int(T.Q4_K), fake, 4, 100, fake, 1, fake, fake, 1 << 20, None) == _lib.VQ_ERR_SHAPE
    assert lib.vq_qmv(int(T.Q4_K), fake, 0, 256, fake, 1, fake, fake, 1 << 20, None) == _lib.VQ_ERR_SHAPE
    assert lib.vq_qmv(int(T.Q4_K), fake, 4, 256, fake, 0, fake, fake, 1 << 20, None) == _lib.VQ_ERR_SHAPE
    assert lib.vq_qmv(int(T.Q4_K), None, 4, 256, fake, 1, fake, fake, 1 << 20, None) == _lib.VQ_ERR_ARG
    assert lib.vq_qmv(int(T.Q4_K), ctypes.c_void_p(0x1008), 4, 256, fake, 1, fake, None, 0, None) == _lib.VQ_ERR_ARG
    assert lib.vq_qmv(int(T.Q4_K), fake, 4, 256, ctypes.c_void_p(0x1004), 1, fake, None, 0, None) == _lib.VQ_ERR_ARG
    assert lib.vq_qmv_packed(int(T.Q4_K), fake, 4, 256, ctypes.c_void_p(0x1001), 1, fake, None) == _lib.VQ_ERR_ARG
    assert lib.vq_qmv_packed(int(T.F32), fake, 4, 256, fake, 1, fake, None) == _lib.VQ_ERR_TYPE
    assert lib.vq_qmv_packed(int(T.Q4_K), fake, 4, 256, None, 1, fake, None) == _lib.VQ_ERR_ARG
    assert lib.vq_quantize_x(fake, 1, 48, fake, fake, None, None) == _lib.VQ_ERR_SHAPE
    assert lib.vq_pack_x(fake, 1, 48, fake, None) == _lib.VQ_ERR_SHAPE
    assert lib.vq_int_partials(int(T.F16), fake, 4, 256, fake, 1, fake, None) == _lib.VQ_ERR_TYPE
    assert lib.vq_argmax_rows(fake, 0, 1, fake, None) == _lib.VQ_ERR_SHAPE
    assert lib.vq_set_iq3s_grid(None) == _lib.VQ_ERR_ARG
    # packed record: cols int8 codes + cols/32 fp32 scales + cols/32 u32 half sums, 16-byte aligned per token
    assert lib.vq_xpack_bytes(5120, 1) == 5120 + 160 * 8
    assert lib.vq_xpack_bytes(96, 1) == 128 and lib.vq_xpack_bytes(96, 3) == 384
    assert lib.vq_xpack_bytes(48, 1) == 0
    assert lib.vq_qmv_workspace_bytes(5120, 8) == 0  # narrow inputs are quantized inside the matvec
    assert lib.vq_qmv_workspace_bytes(17408, 2) == 0  # the FFN down input too
    assert lib.vq_qmv_workspace_bytes(32768, 2) == lib.vq_xpack_bytes(32768, 2)
    assert lib.vq_qmv(int(T.Q4_K), fake, 4, 32768, fake, 1, fake, None, 0, None) == _lib.VQ_ERR_WORKSPACE
    arr = (ctypes.c_void_p * 5)(*([fake] * 5))
    rws = (ctypes.c_int * 5)(*([4] * 5))
    assert lib.vq_qmv_group(int(T.Q4_K), 0, arr, rws, arr, 256, fake, 1, None) == _lib.VQ_ERR_ARG
    assert lib.vq_qmv_group(int(T.Q4_K), 5, arr, rws, arr, 256, fake, 1, None) == _lib.VQ_ERR_ARG
    assert lib.vq_qmv_group(int(T.F32), 2, arr, rws, arr, 256, fake, 1, None) == _lib.VQ_ERR_TYPE
    assert lib.vq_qmv_group(int(T.Q4_K), 2, arr, rws, arr, 100, fake, 1, None) == _lib.VQ_ERR_SHAPE
    assert lib.vq_lmhead_argmax_workspace_bytes(int(T.F16), 4, 256, 1) == 0
    # prefill: the f16-MFMA path (Q3_K-Q6_K) needs the split activations (2 x f16 per element) and more
    assert lib.vq_qgemm_workspace_bytes(int(T.Q6_K), 17408, 5120, 512) >= 4 * 512 * 5120
    assert lib.vq_qgemm_workspace_bytes(int(T.Q3_K), 17408, 5120, 512) >= 4 * 512 * 5120
    assert lib.vq_qgemm_workspace_bytes(int(T.Q2_K), 17408, 5120, 512) >= 4 * 512 * 5120
    assert lib.vq_qgemm_workspace_bytes(int(T.Q8_0), 17408, 5120, 512) == 0
    assert lib.vq_qgemm_workspace_bytes(int(T.IQ4_XS), 17408, 5120, 512) == 0
    assert lib.vq_qgemm_workspace_bytes(int(T.Q4_K), 17408, 5120, 512) >= 4 * 512 * 5120
    assert lib.vq_qgemm_workspace_bytes(int(T.Q4_K), 17408, 5120, 0) == 0
    assert lib.vq_qgemm_ws(int(T.Q4_K), fake, 4, 256, fake, 1, fake, None, 0, None) == _lib.VQ_ERR_WORKSPACE
    assert lib.vq_qgemm_ws(int(T.F32), fake, 4, 256, fake, 1, fake, None, 0, None) == _lib.VQ_ERR_TYPE
    nws = lib.vq_lmhead_argmax_workspace_bytes(int(T.Q6_K), 248320, 5120, 1)
    assert nws >= 8 * 256  # one key per workgroup (one or more per CU) per token
    assert lib.vq_lmhead_argmax(int(T.Q6_K), fake, 248320, 5120, fake, 1, fake, None, fake, nws - 1,
                                None) == _lib.VQ_ERR_WORKSPACE
    assert b"workspace" in lib.vq_status_string(_lib.VQ_ERR_WORKSPACE)


def test_qmv_path_routing(lib):
    """vq_qmv_path: which path vq_qmv takes (host-side; no device needed)."""
    STREAM, I8, F16 = 0, 1, 2
    ws_for = lib.vq_qmv_workspace_bytes_for
    q6, q3, q4 = int(T.Q6_K), int(T.Q3_K), int(T.Q4_K)
    # 5120x17408: the streaming image holds 2 tokens at 17408 columns, so 3..4 tokens take the f16 path
    for ntok, want in ((1, STREAM), (2, STREAM), (3, F16), (4, F16), (8, F16), (16, F16), (17, STREAM)):
        assert lib.vq_qmv_path(q6, 5120, 17408, ntok, ws_for(q6, 5120, 17408, ntok)) == want, ntok
    assert lib.vq_qmv_path(q6, 5120, 17408, 4, 0) == STREAM  # the K-range partials need the workspace
    # 17408x5120: one streaming pass holds 8 tokens, so the f16 path starts at 5
    for ntok, want in ((4, STREAM), (5, F16), (8, F16)):
        assert lib.vq_qmv_path(q3, 17408, 5120, ntok, ws_for(q3, 17408, 5120, ntok)) == want, ntok
    assert lib.vq_qmv_path(q4, 100, 512, 5, 0) == F16  # one K range: no partials, no workspace
    iq, q2, q8 = int(T.IQ4_XS), int(T.Q2_K), int(T.Q8_0)
    assert lib.vq_qmv_path(iq, 5120, 17408, 8, ws_for(iq, 5120, 17408, 8)) == F16  # the IQ types too
    assert lib.vq_qmv_path(iq, 5120, 17408, 8, 0) == STREAM
    assert lib.vq_qmv_path(q2, 5120, 17408, 8, ws_for(q2, 5120, 17408, 8)) == I8  # Q2_K, Q8_0, IQ4_NL: int8 MFMA
    assert lib.vq_qmv_path(q8, 48, 5120, 8, ws_for(q8, 48, 5120, 8)) == I8
    assert lib.vq_qmv_path(q2, 5120, 17408, 5, ws_for(q2, 5120, 17408, 5)) == STREAM
    assert lib.vq_qmv_path(int(T.F32), 64, 64, 8, 1 << 20) == STREAM
    assert lib.vq_qmv_path(99, 64, 256, 1, 0) == -1
    assert lib.vq_qmv_path(q4, 64, 256, 0, 0) == -2
    assert lib.vq_qmv_path(q4, 64, 100, 1, 0) == -2


def test_python_error_mapping(lib):
    with pytest.raises(ValueError):
        _lib.check(_lib.VQ_ERR_SHAPE, "qmv")
    with pytest.raises(RuntimeError, match="qmv failed"):
        _lib.check(_lib.VQ_ERR_WORKSPACE, "qmv")


def test_upload_validation_mirrors_reference():
    # test_phase30_cuda_qmatvec.py:127-134: Q4_0 is rejected, a wrong byte length is rejected.
    with pytest.raises(ValueError):
        runtime._check_upload_args("w", 34, int(T.Q4_0) if hasattr(T, "Q4_0") else 2, 32, 1)
    with pytest.raises(ValueError):
        runtime._check_upload_args("w", 33, int(T.Q8_0), 32, 1)
    with pytest.raises(ValueError):
        runtime._check_upload_args("w", 144, int(T.Q4_K), 128, 1)  # cols not a multiple of 256
    assert runtime._check_upload_args("w", 2 * 144, int(T.Q4_K), 256, 2) == (144, 288)
    with pytest.raises(ValueError):
        runtime._check_qmv_args("w", 256, 0)
    with pytest.raises(ValueError):
        runtime._check_qmv_args("w", 48, 1)


def test_product_does_not_import_oracle():
    for path in (ROOT / "vinf_3080ti_amd").rglob("*.py"):
        text = path.read_text()
        assert "oracle" not in re.findall(r"^\s*(?:from|import)\s+(\w+)", text, re.M), path


# Every runtime method the reference's executor calls on a model whose weights are all resident: the
# QwenGpuExecutor in src/vinf/qwen_gpu.py (load path :575-630 incl. the dynamic weight groups, stats :673,833,
# decode :1263-1286, forward passes) and the backend's stats in src/vinf/qwen_backend.py. A missing name makes
# QwenGpuExecutor(..., runtime=HipWeightRuntime()) fail with AttributeError.
EXECUTOR_RUNTIME_CALLS = (
    "add add_weight_group alloc argmax argmax_rows attention attention_seg buffer_bytes concat_rows conv_update "
    "conv_update_seg copy demote_group device_bytes gated_delta gated_delta_seg gated_rmsnorm kv_append "
    "kv_append_seg map_cost map_range mem_info promote_group qmv read read_floats reserve_ring rmsnorm rope "
    "rope_seg set_arena set_paging set_segments set_stream_order set_weight_space sigmoid_mul silu_mul "
    "split_gated_q staging_bytes streamed_bytes unmap_range upload_gguf_tensor vmm_granularity vram_bytes "
    "weight_groups write zero_range pinned_bytes synchronize"
).split()


def test_hip_weight_runtime_has_every_executor_call():
    missing = [n for n in EXECUTOR_RUNTIME_CALLS
               if not (hasattr(runtime.HipWeightRuntime, n) or hasattr(runtime.Runtime, n))]
    assert missing == []
