"""gfxinfer_amd: MI355X (gfx950) speculative-verify hot path.

Python view of the C ABI declared in include/gfxinfer_amd.h.  The compute lives
in libgfxinfer_amd.so (hand-written HIP for gfx950); this module only loads it,
declares the signatures and offers thin wrappers that mirror the reference
launchers (src/kernels/lowbit_gemv.hip, src/kernels/qwen_ops.hip) with the same
argument meaning and error behaviour: a non-zero status raises GfxinferError
carrying the reference ErrorCode value and message.

There is no fallback: if the library is missing, importing the wrappers fails.
"""
from __future__ import annotations

import ctypes
import os
import re
import subprocess

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
# GFXINFER_AMD_LIBRARY selects another build of the same library (the host-sanitizer
# build of `make -C gfxinfer_amd sanitize`); the default is the in-tree build.
LIBRARY = os.environ.get("GFXINFER_AMD_LIBRARY") or os.path.join(HERE, "libgfxinfer_amd.so")
HEADERS = [os.path.join(ROOT, "include", "gfxinfer_amd.h"),
           os.path.join(ROOT, "include", "gfxinfer_runtime.h")]

# include/gfxinfer/status.h:11-20
OK, INVALID_ARGUMENT, IO_ERROR, CORRUPT_ARTIFACT, UNSUPPORTED, HIP_ERROR, OUT_OF_MEMORY, INTERNAL = range(8)
# include/gfxinfer/artifact.h:26-33
W2G128, W3G128, W4G128 = 1, 2, 3
ERROR_NAMES = {0: "ok", 1: "invalid_argument", 2: "io_error", 3: "corrupt_artifact",
               4: "unsupported", 5: "hip_error", 6: "out_of_memory", 7: "internal"}


class GfxinferError(RuntimeError):
    def __init__(self, code: int, message: str):
        super().__init__(f"{ERROR_NAMES.get(code, code)}: {message}")
        self.code = code
        self.message = message


def build(jobs: int = 8) -> None:
    """Compile libgfxinfer_amd.so for gfx950 in-tree."""
    subprocess.run(["make", "-s", "-C", HERE, f"-j{jobs}"], check=True)


_lib: ctypes.CDLL | None = None

P = ctypes.c_void_p
SZ = ctypes.c_size_t
U32 = ctypes.c_uint32
I32 = ctypes.c_int32
F32 = ctypes.c_float

# name -> (restype, argtypes).  Every function of include/gfxinfer_amd.h.
SIGNATURES: dict[str, tuple] = {
    "gfxinfer_last_error": (ctypes.c_char_p, []),
    "gfxinfer_require_gfx950_device": (I32, [I32]),
    "gfxinfer_packed_row_bytes": (SZ, [I32, SZ]),
    "gfxinfer_tile_group128_for_gfx950": (I32, [I32, P, P, SZ, SZ, P, P]),
    "gfxinfer_untile_group128_for_gfx950": (I32, [I32, P, P, SZ, SZ, P, P]),
    "gfxinfer_launch_quantize_group128_gfx950": (I32, [I32, P, SZ, SZ, P, P, P, P]),
    "gfxinfer_launch_quantize_activation_i4": (I32, [P, P, P, SZ, U32, P]),
    "gfxinfer_launch_quantize_activation_i8": (I32, [P, P, P, SZ, U32, P]),
    "gfxinfer_launch_gfx950_i4_gemm": (I32, [I32, P, P, P, P, P, SZ, SZ, U32, I32, P]),
    "gfxinfer_launch_gfx950_i4_gemm_split": (I32, [I32, P, P, P, P, P, SZ, SZ, U32, U32, P]),
    "gfxinfer_gemm_split_count": (U32, [SZ, SZ, U32]),
    "gfxinfer_launch_gfx950_i4_gemm_half": (I32, [I32, P, P, P, P, P, SZ, SZ, U32, I32, P]),
    "gfxinfer_launch_gfx950_i4_gemm_fused": (I32, [I32, P, SZ, P, P, SZ, U32, I32, P]),
    "gfxinfer_launch_gfx950_i8_gemm": (I32, [I32, P, P, P, P, P, SZ, SZ, U32, P]),
    "gfxinfer_gemm_argmax_workspace_bytes": (SZ, [SZ, U32]),
    "gfxinfer_launch_gfx950_i4_gemm_argmax": (I32, [I32, P, P, P, P, P, SZ, SZ, U32, SZ, P, P, SZ, P, P]),
    "gfxinfer_launch_gfx950_i4_gemm_argmax_no_alloc": (I32, [I32, P, P, P, P, P, SZ, SZ, U32, SZ, P, P, P]),
    "gfxinfer_debug_gemm_partials": (I32, [I32, P, I32, P, SZ, SZ, U32, P, P]),
    "gfxinfer_debug_gemm_family": (I32, [I32, I32, P, P, P, P, P, I32, P, P, U32, SZ, SZ, U32, U32, P]),
    "gfxinfer_debug_stream_read": (I32, [P, SZ, P, U32, P]),
    "gfxinfer_debug_stream_read_oneshot": (I32, [P, SZ, P, U32, P]),
    "gfxinfer_launch_lowbit_row_gather_tiled": (I32, [I32, P, P, P, SZ, SZ, SZ, P]),
    "gfxinfer_launch_lowbit_row_gather_tiled_indirect": (I32, [I32, P, P, P, P, SZ, SZ, P]),
    "gfxinfer_launch_lowbit_row_gather_tiled_batch": (I32, [I32, P, P, P, P, P, P, U32, SZ, SZ, P]),
    "gfxinfer_launch_rms_norm": (I32, [P, P, P, SZ, F32, I32, P]),
    "gfxinfer_launch_rms_norm_batch": (I32, [P, P, P, SZ, U32, F32, I32, P]),
    "gfxinfer_launch_residual_add_rms_norm_batch": (I32, [P, P, P, P, P, SZ, U32, F32, I32, P]),
    "gfxinfer_launch_rms_norm_quantize_i4": (I32, [P, P, P, P, P, SZ, U32, F32, I32, P]),
    "gfxinfer_launch_residual_add_rms_norm_quantize_i4": (I32, [P, P, P, P, P, P, P, SZ, U32, F32, I32, P]),
    "gfxinfer_launch_residual_add_rms_norm_quantize_i4_planes": (I32, [P, P, U32, P, P, P, P, P, SZ, U32, F32, I32, P]),
    "gfxinfer_launch_dual_rms_norm_concat": (I32, [P, P, P, P, P, SZ, F32, I32, P]),
    "gfxinfer_launch_mtp_input_quantize_i4": (I32, [I32, P, P, SZ, U32, P, P, P, P, P, P, P, SZ, F32, I32, P]),
    "gfxinfer_launch_mtp_input_quantize_i4_from_keys": (I32, [I32, P, P, SZ, P, SZ, P, P, P, P, P, P, P, P, SZ, F32, I32, P]),
    "gfxinfer_launch_dual_rms_norm_concat_batch": (I32, [P, P, P, P, P, SZ, U32, F32, I32, P]),
    "gfxinfer_launch_silu_multiply": (I32, [P, P, P, SZ, P]),
    "gfxinfer_launch_silu_multiply_quantize_i4": (I32, [P, P, P, P, SZ, U32, P]),
    "gfxinfer_launch_float_to_half": (I32, [P, P, SZ, P]),
    "gfxinfer_launch_gdn_conv_update_block": (I32, [P, P, P, P, P, P, SZ, U32, P]),
    "gfxinfer_launch_gdn_recurrent_decode_block": (I32, [P, P, P, P, P, P, P, P, P, P, P, P, P, U32, U32, U32, U32, P, P]),
    "gfxinfer_launch_gdn_recurrent_window": (I32, [P, P, P, P, P, P, P, P, P, P, P, U32, U32, U32, U32, P]),
    "gfxinfer_launch_gdn_output_quantize_i4": (I32, [P, P, P, P, P, P, U32, U32, U32, P]),
    "gfxinfer_launch_gdn_conv_window": (I32, [P, P, P, P, P, P, P, P, P, P, P, P, P, P, P, U32, U32, U32, U32, P]),
    "gfxinfer_launch_gdn_restore_prefix_all": (I32, [P, P, P, P, P, P, SZ, U32, U32, U32, U32, U32, U32, P]),
    "gfxinfer_launch_qk_rms_norm_rope_block": (I32, [P, P, P, SZ, SZ, P, P, P, SZ, SZ, SZ, SZ, ctypes.c_uint64, U32, F32, P]),
    "gfxinfer_launch_qk_rms_norm_rope_block_indirect_position": (I32, [P, P, P, SZ, SZ, P, P, P, SZ, SZ, SZ, SZ, P, U32, F32, P]),
    "gfxinfer_launch_qk_rms_norm_rope_kv_append_block": (I32, [P, P, P, SZ, SZ, P, P, P, SZ, SZ, SZ, SZ, P, P, P, SZ, ctypes.c_uint64, U32, F32, P]),
    "gfxinfer_launch_qk_rms_norm_rope_kv_append_block_indirect_position": (I32, [P, P, P, SZ, SZ, P, P, P, SZ, SZ, SZ, SZ, P, P, P, SZ, P, U32, F32, P]),
    "gfxinfer_launch_kv_append_block": (I32, [P, P, P, P, SZ, SZ, U32, SZ, P]),
    "gfxinfer_launch_kv_append_block_indirect_position": (I32, [P, P, P, P, P, SZ, U32, SZ, P]),
    "gfxinfer_launch_argmax_batch": (I32, [P, P, SZ, SZ, U32, P]),
    "gfxinfer_launch_argmax_mapped": (I32, [P, P, P, SZ, P]),
    "gfxinfer_attention_workspace_bytes": (SZ, [U32, U32, U32, SZ]),
    "gfxinfer_launch_gated_attention_decode_block": (I32, [P, P, P, P, P, SZ, SZ, U32, U32, U32, U32, P, SZ, P]),
    "gfxinfer_launch_gated_attention_decode_block_indirect_position": (I32, [P, P, P, P, P, P, SZ, U32, U32, U32, U32, P, SZ, P]),
    "gfxinfer_launch_gated_attention_decode_block_quantize_i4": (I32, [P, P, P, P, P, P, P, SZ, SZ, U32, U32, U32, U32, P, SZ, P]),
    "gfxinfer_launch_gated_attention_decode_block_quantize_i4_indirect_position": (I32, [P, P, P, P, P, P, P, P, SZ, U32, U32, U32, U32, P, SZ, P]),
    "gfxinfer_launch_qk_rms_norm_rope_kv_append_attention_quantize_i4": (I32, [P, P, SZ, P, P, SZ, P, SZ, F32, P, P, P, P, P, P, P, SZ, SZ, U32, U32, U32, U32, P, SZ, P]),
    "gfxinfer_launch_qk_rms_norm_rope_kv_append_attention_quantize_i4_indirect_position": (I32, [P, P, SZ, P, P, SZ, P, SZ, F32, P, P, P, P, P, P, P, P, SZ, U32, U32, U32, U32, P, SZ, P]),
    "gfxinfer_rope_table_bytes": (SZ, [SZ, SZ]),
    "gfxinfer_launch_rope_table": (I32, [P, SZ, SZ, F32, P]),
    "gfxinfer_fused_rope_attention_supported": (I32, [U32, U32, U32, U32]),
    "gfxinfer_launch_gdn_conv_update": (I32, [P, P, P, P, SZ, P]),
    "gfxinfer_launch_gdn_recurrent_decode": (I32, [P, P, P, P, P, P, P, P, P, U32, U32, U32, P, P]),
    "gfxinfer_launch_gdn_restore_prefix": (I32, [P, P, P, P, P, P, SZ, U32, U32, U32, U32, P]),
    "gfxinfer_launch_kv_append": (I32, [P, P, P, P, SZ, SZ, SZ, P]),
    "gfxinfer_launch_gated_attention_decode": (I32, [P, P, P, P, P, SZ, SZ, U32, U32, U32, P, SZ, P]),
    "gfxinfer_qwen38_scratch_bytes": (SZ, [U32, SZ]),
    "gfxinfer_qwen38_bind_scratch": (I32, [P, P, SZ, U32, SZ]),
    "gfxinfer_qwen38_unbind_scratch": (I32, [P]),
    "gfxinfer_qwen38_launch_gated_attention_decode": (I32, [P, P, P, P, P, SZ, SZ, P]),
    "gfxinfer_qwen38_launch_gated_attention_decode_block": (I32, [P, P, P, P, P, SZ, SZ, U32, P]),
    "gfxinfer_qwen38_launch_gated_attention_decode_block_indirect_position": (I32, [P, P, P, P, P, P, SZ, U32, P]),
    "gfxinfer_qwen38_launch_gdn_recurrent_decode_block": (I32, [P] * 13 + [U32, P]),
    "gfxinfer_qwen38_launch_gdn_recurrent_decode": (I32, [P] * 10),
    "gfxinfer_launch_argmax": (I32, [P, P, SZ, P]),
    # include/gfxinfer_runtime.h
    "gfxinfer_model_spec_qwen38_27b": (None, [P]),
    "gfxinfer_model_spec_qwen38_reference": (None, [P]),
    "gfxinfer_model_spec_tensor_count": (SZ, [P]),
    "gfxinfer_model_spec_tensor": (I32, [P, SZ, P]),
    "gfxinfer_model_create_synthetic": (I32, [P, ctypes.c_uint64, I32, P]),
    "gfxinfer_model_destroy": (None, [P]),
    "gfxinfer_model_stream": (P, [P]),
    "gfxinfer_model_weight_bytes": (SZ, [P]),
    "gfxinfer_model_find_tensor": (I32, [P, ctypes.c_char_p, P]),
    "gfxinfer_model_copy_tensor": (I32, [P, ctypes.c_char_p, I32, P, SZ]),
    "gfxinfer_artifact_open": (I32, [ctypes.c_char_p, I32, P]),
    "gfxinfer_artifact_close": (None, [P]),
    "gfxinfer_artifact_get_identity": (I32, [P, P]),
    "gfxinfer_artifact_tensor_count": (SZ, [P]),
    "gfxinfer_artifact_tensor_at": (I32, [P, SZ, P]),
    "gfxinfer_artifact_find": (I32, [P, ctypes.c_char_p, P]),
    "gfxinfer_artifact_bytes": (P, [P, ctypes.c_uint64, ctypes.c_uint64]),
    "gfxinfer_crc64_ecma": (ctypes.c_uint64, [ctypes.c_uint64, P, SZ]),
    "gfxinfer_artifact_resource": (I32, [P, ctypes.c_char_p, ctypes.POINTER(P), ctypes.POINTER(ctypes.c_uint64)]),
    "gfxinfer_tokenizer_create": (I32, [P, SZ, ctypes.POINTER(P)]),
    "gfxinfer_tokenizer_destroy": (None, [P]),
    "gfxinfer_tokenizer_vocabulary_size": (SZ, [P]),
    "gfxinfer_tokenizer_encode": (I32, [P, ctypes.c_char_p, SZ, P, SZ, ctypes.POINTER(SZ)]),
    "gfxinfer_tokenizer_decode": (I32, [P, P, SZ, P, SZ, ctypes.POINTER(SZ)]),
    "gfxinfer_render_chat_prompt": (I32, [ctypes.c_char_p, SZ, P, SZ, ctypes.POINTER(SZ)]),
    "gfxinfer_retile_gfx12_for_gfx950": (I32, [I32, P, SZ, P]),
    "gfxinfer_model_create_from_artifact": (I32, [P, ctypes.c_char_p, I32, I32, P]),
    "gfxinfer_model_write_artifact": (I32, [P, ctypes.c_char_p, ctypes.c_char_p, P, SZ]),
    "gfxinfer_session_create": (I32, [P, P, P]),
    "gfxinfer_session_destroy": (None, [P]),
    "gfxinfer_session_greedy_step": (I32, [P, U32, P]),
    "gfxinfer_session_block_step": (I32, [P, P, SZ, P]),
    "gfxinfer_session_mtp_draft": (I32, [P, U32, P]),
    "gfxinfer_session_speculative_step": (I32, [P, U32, SZ, P]),
    "gfxinfer_session_speculative_step_forced": (I32, [P, U32, SZ, U32, P]),
    "gfxinfer_session_speculative_step_planted": (I32, [P, U32, SZ, P, P]),
    "gfxinfer_session_position": (SZ, [P]),
    "gfxinfer_session_mtp_position": (SZ, [P]),
    "gfxinfer_session_get_summary": (I32, [P, P]),
    "gfxinfer_session_copy_buffer": (I32, [P, ctypes.c_char_p, SZ, P, SZ]),
    "gfxinfer_session_buffer_bytes": (SZ, [P, ctypes.c_char_p]),
    "gfxinfer_session_set_layer_trace": (I32, [P, P, SZ]),
    "gfxinfer_session_layer_trace_bytes": (SZ, [P]),
    "gfxinfer_session_prefill": (I32, [P, P, SZ, I32, P]),
    "gfxinfer_session_generate": (I32, [P, P, SZ, P, P, P, P]),
    "gfxinfer_depth_policy_create": (I32, [U32, P]),
    "gfxinfer_depth_policy_destroy": (None, [P]),
    "gfxinfer_depth_policy_choose": (U32, [P, U32]),
    "gfxinfer_depth_policy_record": (I32, [P, U32, U32, ctypes.c_double]),
}


class FusedMatrix(ctypes.Structure):
    """gfxinfer_fused_matrix (lowbit_gemv.h:128-133 Gfx12I4FusedMatrix)."""
    _fields_ = [("tiled_weights", P), ("tiled_weight_scales", P), ("output", P), ("rows", SZ)]


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not os.path.exists(LIBRARY):
            raise RuntimeError(
                f"{LIBRARY} is not built; run __graft_entry__.build() (hipcc for gfx950)")
        # PyTorch-ROCm ships its own libamdhip64 (soname libamdhip64.so.7).  Loading it
        # first lets this library bind to that same HIP runtime; loading
        # /opt/rocm's copy first would put two HIP runtimes in one process.
        try:
            import torch  # noqa: F401
        except ImportError:
            pass
        L = ctypes.CDLL(LIBRARY)
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _lib = L
    return _lib


def header_functions() -> list[str]:
    """Names of every function declared in include/*.h."""
    text = "\n".join(open(h).read() for h in HEADERS)
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(gfxinfer_[a-z0-9_]+)\s*\(", text)))


def last_error() -> str:
    return lib().gfxinfer_last_error().decode()


def check(status: int) -> None:
    if status != OK:
        raise GfxinferError(status, last_error())


def _p(x) -> int | None:
    """Device/host address of a torch tensor, numpy array or raw int."""
    if x is None:
        return None
    if isinstance(x, int):
        return x
    if hasattr(x, "data_ptr"):
        return x.data_ptr()
    return x.ctypes.data


def _stream(stream) -> int | None:
    if stream is None:
        import torch
        return torch.cuda.current_stream().cuda_stream
    if isinstance(stream, int):
        return stream
    return stream.cuda_stream


# ---- wrappers (reference launcher names, lowbit_gemv.h) ---------------------

def launch_quantize_activation_i4(x, packed, scales, columns, batch, stream=None):
    check(lib().gfxinfer_launch_quantize_activation_i4(_p(x), _p(packed), _p(scales), columns, batch, _stream(stream)))


def launch_quantize_activation_i8(x, codes, scales, columns, batch, stream=None):
    check(lib().gfxinfer_launch_quantize_activation_i8(_p(x), _p(codes), _p(scales), columns, batch, _stream(stream)))


def launch_quantize_group128(fmt, weights, rows, columns, codes, scales, flag=None, stream=None):
    check(lib().gfxinfer_launch_quantize_group128_gfx950(fmt, _p(weights), rows, columns, _p(codes), _p(scales), _p(flag), _stream(stream)))


def launch_i4_gemm(fmt, w, ws, a, as_, out, rows, columns, batch, stream=None):
    check(lib().gfxinfer_launch_gfx950_i4_gemm(fmt, _p(w), _p(ws), _p(a), _p(as_), _p(out), rows, columns, batch, 1, _stream(stream)))


def launch_i4_gemm_split(fmt, w, ws, a, as_, planes, rows, columns, batch, splits, stream=None):
    """Split-K GEMM: `splits` fp32 planes [splits, batch, rows] whose sum is the product."""
    check(lib().gfxinfer_launch_gfx950_i4_gemm_split(fmt, _p(w), _p(ws), _p(a), _p(as_), _p(planes), rows, columns, batch, splits, _stream(stream)))


def gemm_split_count(rows, columns, batch):
    return int(lib().gfxinfer_gemm_split_count(rows, columns, batch))


def launch_i4_gemm_half(fmt, w, ws, a, as_, out, rows, columns, batch, stream=None):
    check(lib().gfxinfer_launch_gfx950_i4_gemm_half(fmt, _p(w), _p(ws), _p(a), _p(as_), _p(out), rows, columns, batch, 1, _stream(stream)))


def launch_i4_gemm_fused(fmt, matrices, a, as_, columns, batch, stream=None):
    """matrices: list of (weights, scales, output, rows)."""
    arr = (FusedMatrix * len(matrices))(*[FusedMatrix(_p(w), _p(s), _p(o), r) for (w, s, o, r) in matrices])
    check(lib().gfxinfer_launch_gfx950_i4_gemm_fused(fmt, ctypes.cast(arr, P), len(matrices), _p(a), _p(as_), columns, batch, 1, _stream(stream)))


def launch_i8_gemm(fmt, w, ws, a, as_, out, rows, columns, batch, stream=None):
    check(lib().gfxinfer_launch_gfx950_i8_gemm(fmt, _p(w), _p(ws), _p(a), _p(as_), _p(out), rows, columns, batch, _stream(stream)))


def debug_gemm_partials(fmt, w, abits, a, rows, columns, batch, partials, stream=None):
    check(lib().gfxinfer_debug_gemm_partials(fmt, _p(w), abits, _p(a), rows, columns, batch, _p(partials), _stream(stream)))


GEMM_MFMA, GEMM_DOT = 1, 2


def debug_gemm_family(family, fmt, w, ws, a, as_, rows, columns, batch, out=None, half_output=False,
                      partials=None, argmax_keys=None, argmax_rows=0, splits=1, stream=None):
    """One A4 GEMM launch through a named kernel family (GEMM_MFMA or GEMM_DOT); returns the status."""
    return int(lib().gfxinfer_debug_gemm_family(family, fmt, _p(w), _p(ws), _p(a), _p(as_), _p(out),
                                                1 if half_output else 0, _p(partials), _p(argmax_keys),
                                                argmax_rows, rows, columns, batch, splits, _stream(stream)))


def debug_stream_read(data, nbytes, sink, workgroups, stream=None):
    check(lib().gfxinfer_debug_stream_read(_p(data), nbytes, _p(sink), workgroups, _stream(stream)))


def debug_stream_read_oneshot(data, nbytes, sink, loads_per_lane, stream=None):
    check(lib().gfxinfer_debug_stream_read_oneshot(_p(data), nbytes, _p(sink), loads_per_lane, _stream(stream)))


def launch_row_gather_tiled(fmt, w, ws, out, row, rows, columns, stream=None):
    check(lib().gfxinfer_launch_lowbit_row_gather_tiled(fmt, _p(w), _p(ws), _p(out), row, rows, columns, _stream(stream)))


def launch_row_gather_tiled_batch(fmt, w, ws, out, host_rows, first_row, rest_rows, count, rows, columns,
                                  stream=None):
    """host_rows: a sequence of ints or None; first_row / rest_rows: device uint32 tensors or None."""
    array = (ctypes.c_uint32 * count)(*host_rows) if host_rows is not None else None
    host = ctypes.cast(array, ctypes.c_void_p) if array is not None else None
    check(lib().gfxinfer_launch_lowbit_row_gather_tiled_batch(fmt, _p(w), _p(ws), _p(out), host, _p(first_row),
                                                              _p(rest_rows), count, rows, columns,
                                                              _stream(stream)))


def launch_row_gather_tiled_indirect(fmt, w, ws, out, row_ptr, rows, columns, stream=None):
    check(lib().gfxinfer_launch_lowbit_row_gather_tiled_indirect(fmt, _p(w), _p(ws), _p(out), _p(row_ptr), rows, columns, _stream(stream)))


# ---- host-side layout (numpy) -------------------------------------------------

def packed_row_bytes(fmt: int, columns: int) -> int:
    return int(lib().gfxinfer_packed_row_bytes(fmt, columns))


def tile_bytes(fmt: int, rows: int, columns: int) -> int:
    return rows * columns * {W2G128: 2, W3G128: 3}.get(fmt, 4) // 8


def tile_group128(fmt, packed_codes, scales, rows, columns):
    """Reference-packed codes + float scales -> (tiled codes, fp16 scale bits)."""
    import numpy as np
    packed_codes = np.ascontiguousarray(packed_codes, dtype=np.uint8)
    scales = np.ascontiguousarray(scales, dtype=np.float32)
    codes = np.zeros(tile_bytes(fmt, rows, columns), dtype=np.uint8)
    tscales = np.zeros(rows * (columns // 128), dtype=np.uint16)
    check(lib().gfxinfer_tile_group128_for_gfx950(fmt, _p(packed_codes), _p(scales), rows, columns, _p(codes), _p(tscales)))
    return codes, tscales


def untile_group128(fmt, codes, tscales, rows, columns):
    """Tiled codes (+ fp16 scales) -> (int8 weights [rows, columns], fp16 scale bits [rows, G])."""
    import numpy as np
    codes = np.ascontiguousarray(codes, dtype=np.uint8)
    w = np.empty((rows, columns), dtype=np.int8)
    s = np.empty((rows, columns // 128), dtype=np.uint16)
    ts = None if tscales is None else np.ascontiguousarray(tscales, dtype=np.uint16)
    check(lib().gfxinfer_untile_group128_for_gfx950(fmt, _p(codes), _p(ts), rows, columns, _p(w), _p(s) if ts is not None else None))
    return w, s
