"""numpy binding of the CPU oracle (liboracle.so) and of the reference quantizer
compiled in place (_ref/libgfxref.so).

TEST INFRASTRUCTURE ONLY.  Imported by tests/, by __graft_entry__.smoke() and by
bench.py's cpu_baseline leg, always as the checker; the product never loads it.
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
W2, W3, W4 = 1, 2, 3
GROUP = 128

_lib = None
_ref = None


def build(reference: bool = False) -> None:
    """Compile liboracle.so (and _ref/ when the reference tree is present)."""
    targets = ["all"] + (["ref"] if reference else [])
    subprocess.run(["make", "-s", "-C", HERE] + targets, check=True)


def lib() -> ctypes.CDLL:
    """liboracle.so, or the build GFXINFER_ORACLE_LIBRARY names (the sanitizer build of
    `make -C oracle sanitize`)."""
    global _lib
    if _lib is None:
        path = os.environ.get("GFXINFER_ORACLE_LIBRARY") or os.path.join(HERE, "liboracle.so")
        if not os.path.exists(path):
            build()
        _lib = ctypes.CDLL(path)
        _declare(_lib)
    return _lib


NATIVE_FLAGS = ["-O3", "-march=native", "-std=c11", "-fPIC", "-fopenmp", "-ffp-contract=off"]


def use_native_build(directory: str) -> str:
    """Compile oracle.c for this host's CPU (gcc with NATIVE_FLAGS) into `directory` and
    route every later call through that build; returns the compile command.  The CPU
    baseline uses it on the machine it runs on, so -march=native matches that CPU."""
    global _lib
    path = os.path.join(directory, "liboracle_native.so")
    cmd = ["gcc"] + NATIVE_FLAGS + ["-shared", os.path.join(HERE, "oracle.c"), "-o", path, "-lm"]
    subprocess.run(cmd, check=True)
    native = ctypes.CDLL(path)
    _declare(native)
    _lib = native
    return " ".join(["gcc"] + NATIVE_FLAGS)


def ref_lib() -> ctypes.CDLL | None:
    """The reference's own quantizer, or None when _ref/ was not built."""
    global _ref
    if _ref is None:
        path = os.path.join(HERE, "_ref", "libgfxref.so")
        if not os.path.exists(path):
            return None
        _ref = ctypes.CDLL(path)
        _ref.ref_quantize_group128.restype = ctypes.c_int
        _ref.ref_quantize_group128.argtypes = [P, ctypes.c_size_t, ctypes.c_size_t, ctypes.c_int, P, P]
        _ref.ref_dequantize_group128.restype = ctypes.c_int
        _ref.ref_dequantize_group128.argtypes = [P, P, ctypes.c_size_t, ctypes.c_size_t, ctypes.c_int, P]
        _ref.ref_packed_row_bytes.restype = ctypes.c_size_t
        _ref.ref_packed_row_bytes.argtypes = [ctypes.c_int, ctypes.c_size_t]
        _ref.ref_tile_group128_for_gfx12.restype = ctypes.c_int
        _ref.ref_tile_group128_for_gfx12.argtypes = [P, P, ctypes.c_size_t, ctypes.c_size_t, ctypes.c_int, P, P]
        _ref.ref_write_artifact.restype = ctypes.c_int
        _ref.ref_write_artifact.argtypes = [ctypes.c_char_p] * 5 + [ctypes.c_size_t] + [P] * 9
        _ref.ref_open_artifact.restype = ctypes.c_int
        _ref.ref_open_artifact.argtypes = [ctypes.c_char_p, ctypes.c_int, P]
        _ref.ref_crc64_ecma.restype = ctypes.c_uint64
        _ref.ref_crc64_ecma.argtypes = [P, ctypes.c_size_t]
    return _ref


def ref_write_artifact(path: str, identity: tuple, tensors: list) -> int:
    """The reference ArtifactWriter::write (artifact.cpp:427-545) on `tensors`: dicts with
    name, dtype, quantization, dims, data (bytes-like), aux (bytes-like or None)."""
    R = ref_lib()
    n = len(tensors)
    keep = []
    def arr(values, ctype):
        a = (ctype * len(values))(*values)
        keep.append(a)
        return ctypes.cast(a, P)
    names = [t["name"].encode() for t in tensors]
    name_arr = (ctypes.c_char_p * n)(*names)
    dims = []
    for t in tensors:
        d = list(t["dims"]) + [0] * (4 - len(t["dims"]))
        dims += d
    datas = [np.ascontiguousarray(np.frombuffer(bytes(t["data"]), np.uint8)) for t in tensors]
    auxs = [None if t.get("aux") is None else np.ascontiguousarray(np.frombuffer(bytes(t["aux"]), np.uint8))
            for t in tensors]
    keep += datas + [a for a in auxs if a is not None]
    data_ptrs = (P * n)(*[d.ctypes.data for d in datas])
    aux_ptrs = (P * n)(*[None if a is None else a.ctypes.data for a in auxs])
    return R.ref_write_artifact(
        str(path).encode(), *[x.encode() for x in identity], n, ctypes.cast(name_arr, P),
        arr([t["dtype"] for t in tensors], ctypes.c_int), arr([t["quantization"] for t in tensors], ctypes.c_int),
        arr([len(t["dims"]) for t in tensors], ctypes.c_int), arr(dims, ctypes.c_uint64),
        ctypes.cast(data_ptrs, P), arr([d.nbytes for d in datas], ctypes.c_uint64),
        ctypes.cast(aux_ptrs, P), arr([0 if a is None else a.nbytes for a in auxs], ctypes.c_uint64))


def ref_open_artifact(path: str, verify: bool = True) -> tuple:
    """The reference ArtifactView::open: (status code, tensor count)."""
    count = ctypes.c_size_t(0)
    rc = ref_lib().ref_open_artifact(str(path).encode(), int(verify), ctypes.byref(count))
    return rc, count.value


def ref_tile_gfx12(codes: np.ndarray, scales: np.ndarray, rows: int, cols: int, fmt: int):
    """The reference tile_group128_for_gfx12 (quantization.cpp:253-318)."""
    out_codes = np.empty(codes.size, np.uint8)
    out_scales = np.empty(scales.size, np.float32)
    rc = ref_lib().ref_tile_group128_for_gfx12(ptr(np.ascontiguousarray(codes, np.uint8)),
                                               ptr(np.ascontiguousarray(scales, np.float32)),
                                               rows, cols, fmt, ptr(out_codes), ptr(out_scales))
    if rc != 0:
        raise RuntimeError(f"reference gfx12 tiling failed: {rc}")
    return out_codes, out_scales


P = ctypes.c_void_p
SZ = ctypes.c_size_t
U = ctypes.c_uint
F = ctypes.c_float
I = ctypes.c_int


def _declare(L: ctypes.CDLL) -> None:
    sig = {
        "orc_f32_to_f16": (ctypes.c_uint16, [F]),
        "orc_f16_to_f32": (F, [ctypes.c_uint16]),
        "orc_f32_to_f16_array": (None, [P, P, SZ]),
        "orc_packed_row_bytes": (SZ, [I, SZ]),
        "orc_quantize_group128": (I, [P, SZ, SZ, I, P, P]),
        "orc_unpack_weights": (None, [P, SZ, SZ, I, P]),
        "orc_quantize_activation_i4": (I, [P, P, P, SZ, U]),
        "orc_quantize_activation_i8": (I, [P, P, P, SZ, U]),
        "orc_unpack_a4": (None, [P, SZ, U, P]),
        "orc_gemm_partials": (None, [P, P, SZ, SZ, U, P]),
        "orc_gemm_epilogue": (None, [P, P, P, SZ, SZ, U, P]),
        "orc_gemm_epilogue_ranges": (None, [P, P, P, SZ, SZ, U, U, P]),
        "orc_dequant_dot_gemv": (None, [P, P, P, P, SZ, SZ, U, P]),
        "orc_dequant_dot_gemv_packed": (None, [P, I, P, P, P, SZ, SZ, U, P]),
        "orc_max_threads": (I, []),
        "orc_rms_norm": (None, [P, P, P, SZ, U, F, I]),
        "orc_residual_add_rms_norm": (None, [P, P, P, P, P, SZ, U, F, I]),
        "orc_dual_rms_norm_concat": (None, [P, P, P, P, P, SZ, F, I]),
        "orc_silu_multiply_quantize_i4": (I, [P, P, P, P, SZ, U]),
        "orc_silu_multiply": (None, [P, P, P, SZ]),
        "orc_synthetic_values": (None, [ctypes.c_uint64, SZ, SZ, F, F, P]),
        "orc_gdn_conv_update": (None, [P, P, P, P, P, P, SZ, U]),
        "orc_gdn_recurrent": (None, [P, P, P, P, P, P, P, P, P, P, P, P, P, U, U, U, U]),
        "orc_gdn_restore_conv": (None, [P, P, SZ, U]),
        "orc_gdn_restore_recurrent": (None, [P, P, P, P, U, U, U, U]),
        "orc_head_norm_rope": (None, [P, SZ, P, P, SZ, SZ, SZ, ctypes.c_uint64, U, F]),
        "orc_kv_append": (None, [P, P, P, P, SZ, SZ, U]),
        "orc_gated_attention": (None, [P, P, P, P, P, SZ, U, U, U, U, F]),
        "orc_argmax": (None, [P, SZ, SZ, U, P, P]),
        "orc_accept": (SZ, [P, P, SZ]),
    }
    for name, (res, args) in sig.items():
        fn = getattr(L, name)
        fn.restype = res
        fn.argtypes = args


def ptr(a: np.ndarray | None):
    """A ctypes pointer to `a`'s data that holds a reference to `a`, so that a temporary
    passed as ptr(np.empty(...)) or ptr(np.ascontiguousarray(x)) stays alive until the
    call it is an argument of returns."""
    if a is None:
        return None
    assert a.flags["C_CONTIGUOUS"]
    return a.ctypes.data_as(ctypes.c_void_p)


# ---- fp16 / bf16 ------------------------------------------------------------

def f32_to_f16_bits(x: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.empty(x.shape, dtype=np.uint16)
    lib().orc_f32_to_f16_array(ptr(x), ptr(out), x.size)
    return out


def f16_bits_to_f32(x: np.ndarray) -> np.ndarray:
    return np.ascontiguousarray(x, dtype=np.uint16).view(np.float16).astype(np.float32)


# ---- weight quantizer -------------------------------------------------------

def packed_row_bytes(fmt: int, columns: int) -> int:
    return int(lib().orc_packed_row_bytes(fmt, columns))


def quantize_group128(w: np.ndarray, fmt: int):
    """Returns (status, codes [N, row_bytes] uint8, scales [N, G] float32)."""
    w = np.ascontiguousarray(w, dtype=np.float32)
    rows, cols = w.shape
    codes = np.zeros((rows, max(1, packed_row_bytes(fmt, cols))), dtype=np.uint8)
    scales = np.zeros((rows, max(1, cols // GROUP)), dtype=np.float32)
    status = lib().orc_quantize_group128(ptr(w), rows, cols, fmt, ptr(codes), ptr(scales))
    return int(status), codes, scales


def ref_quantize_group128(w: np.ndarray, fmt: int):
    R = ref_lib()
    if R is None:
        return None
    w = np.ascontiguousarray(w, dtype=np.float32)
    rows, cols = w.shape
    codes = np.zeros((rows, max(1, int(R.ref_packed_row_bytes(fmt, cols)))), dtype=np.uint8)
    scales = np.zeros((rows, max(1, cols // GROUP)), dtype=np.float32)
    status = R.ref_quantize_group128(ptr(w), rows, cols, fmt, ptr(codes), ptr(scales))
    return int(status), codes, scales


def unpack_weights(codes: np.ndarray, rows: int, cols: int, fmt: int) -> np.ndarray:
    codes = np.ascontiguousarray(codes, dtype=np.uint8)
    out = np.empty((rows, cols), dtype=np.int8)
    lib().orc_unpack_weights(ptr(codes), rows, cols, fmt, ptr(out))
    return out


# ---- activation quantizers --------------------------------------------------

def quantize_activation_i4(x16: np.ndarray):
    x16 = np.ascontiguousarray(x16, dtype=np.uint16)
    B, K = x16.shape
    packed = np.zeros((B, K // 2), dtype=np.uint8)
    scales = np.zeros((B, K // GROUP), dtype=np.uint16)
    st = lib().orc_quantize_activation_i4(ptr(x16), ptr(packed), ptr(scales), K, B)
    assert st == 0, st
    return packed, scales


def quantize_activation_i8(x16: np.ndarray):
    x16 = np.ascontiguousarray(x16, dtype=np.uint16)
    B, K = x16.shape
    codes = np.zeros((B, K), dtype=np.int8)
    scales = np.zeros((B, K // GROUP), dtype=np.uint16)
    st = lib().orc_quantize_activation_i8(ptr(x16), ptr(codes), ptr(scales), K, B)
    assert st == 0, st
    return codes, scales


def unpack_a4(packed: np.ndarray, K: int) -> np.ndarray:
    packed = np.ascontiguousarray(packed, dtype=np.uint8)
    B = packed.shape[0]
    out = np.empty((B, K), dtype=np.int8)
    lib().orc_unpack_a4(ptr(packed), K, B, ptr(out))
    return out


# ---- GEMM -------------------------------------------------------------------

def gemm_partials(w: np.ndarray, a: np.ndarray) -> np.ndarray:
    """int32 P[B, N, G] from signed int8 w [N, K] and a [B, K]."""
    w = np.ascontiguousarray(w, dtype=np.int8)
    a = np.ascontiguousarray(a, dtype=np.int8)
    N, K = w.shape
    B = a.shape[0]
    out = np.empty((B, N, K // GROUP), dtype=np.int32)
    lib().orc_gemm_partials(ptr(w), ptr(a), N, K, B, ptr(out))
    return out


def gemm_epilogue(partials: np.ndarray, ws16: np.ndarray, as16: np.ndarray) -> np.ndarray:
    partials = np.ascontiguousarray(partials, dtype=np.int32)
    ws16 = np.ascontiguousarray(ws16, dtype=np.uint16)
    as16 = np.ascontiguousarray(as16, dtype=np.uint16)
    B, N, G = partials.shape
    out = np.empty((B, N), dtype=np.float32)
    lib().orc_gemm_epilogue(ptr(partials), ptr(ws16), ptr(as16), N, G * GROUP, B, ptr(out))
    return out


def gemm_epilogue_ranges(partials: np.ndarray, ws16: np.ndarray, as16: np.ndarray,
                         splits: int = 1) -> np.ndarray:
    """fp32 [splits, B, N]: the epilogue cut into splits and ranges of K, the order in
    which the library's GEMMs add the group partials (splits = 1 -> [1, B, N])."""
    partials = np.ascontiguousarray(partials, dtype=np.int32)
    ws16 = np.ascontiguousarray(ws16, dtype=np.uint16)
    as16 = np.ascontiguousarray(as16, dtype=np.uint16)
    B, N, G = partials.shape
    out = np.empty((splits, B, N), dtype=np.float32)
    lib().orc_gemm_epilogue_ranges(ptr(partials), ptr(ws16), ptr(as16), N, G * GROUP, B, splits, ptr(out))
    return out


def dequant_dot_gemv_packed(codes, fmt, ws, a, as16, N, K):
    codes = np.ascontiguousarray(codes, dtype=np.uint8)
    ws = np.ascontiguousarray(ws, dtype=np.float32)
    a = np.ascontiguousarray(a, dtype=np.int8)
    as16 = np.ascontiguousarray(as16, dtype=np.uint16)
    B = a.shape[0]
    out = np.empty((B, N), dtype=np.float32)
    lib().orc_dequant_dot_gemv_packed(ptr(codes), fmt, ptr(ws), ptr(a), ptr(as16), N, K, B, ptr(out))
    return out


def max_threads() -> int:
    return int(lib().orc_max_threads())


# ---- synthetic checkpoint generator -----------------------------------------
# CPU restatement of the counter-based generator of gfxinfer_model_create_synthetic
# (gfxinfer_amd/csrc/model.hip): key = splitmix64(seed ^ fnv1a64(name)); element i
# is mean + float(n_i) * (sigma * 2^-16) in fp32, n_i = the sum of the twelve 16-bit
# fields of splitmix64(key + 3i + j), j = 0..2, plus 6 - 6 * 65536 (an exact
# Irwin-Hall(12) numerator).  Not a reference algorithm: it only has to agree with
# the device generator, which the runtime tests check bit for bit.

_M64 = np.uint64(0xFFFFFFFFFFFFFFFF)


def _splitmix64(x: np.ndarray) -> np.ndarray:
    with np.errstate(over="ignore"):
        z = x + np.uint64(0x9E3779B97F4A7C15)
        z = (z ^ (z >> np.uint64(30))) * np.uint64(0xBF58476D1CE4E5B9)
        z = (z ^ (z >> np.uint64(27))) * np.uint64(0x94D049BB133111EB)
        return z ^ (z >> np.uint64(31))


def name_hash(name: str) -> int:
    h = 1469598103934665603
    for c in name.encode():
        h ^= c
        h = (h * 1099511628211) & 0xFFFFFFFFFFFFFFFF
    return h


def synthetic_values_c(seed: int, name: str, count: int, sigma: float, mean: float,
                       first: int = 0) -> np.ndarray:
    """synthetic_values computed by liboracle.so (OpenMP): the same values, for the
    full-width model tensors where the numpy form is slow."""
    out = np.empty(count, dtype=np.float32)
    key = (np.uint64(seed) ^ np.uint64(name_hash(name)))
    lib().orc_synthetic_values(ctypes.c_uint64(int(key)), first, count, ctypes.c_float(sigma),
                               ctypes.c_float(mean), ptr(out))
    return out


def synthetic_values(seed: int, name: str, count: int, sigma: float, mean: float,
                     first: int = 0) -> np.ndarray:
    key = _splitmix64(np.array([np.uint64(seed) ^ np.uint64(name_hash(name))], dtype=np.uint64))[0]
    idx = np.arange(first, first + count, dtype=np.uint64)
    total = np.zeros(count, dtype=np.int64)
    with np.errstate(over="ignore"):
        for j in range(3):
            h = _splitmix64(key + np.uint64(3) * idx + np.uint64(j))
            for shift in (0, 16, 32, 48):
                total += ((h >> np.uint64(shift)) & np.uint64(0xFFFF)).astype(np.int64)
    n = (total + 6 - 6 * 65536).astype(np.float32)
    scale = np.float32(sigma) * np.float32(2.0 ** -16)
    return (np.float32(mean) + n * scale).astype(np.float32)


def f32_to_bf16_bits(x: np.ndarray) -> np.ndarray:
    u = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32).astype(np.uint64)
    return ((u + np.uint64(0x7FFF) + ((u >> np.uint64(16)) & np.uint64(1))) >> np.uint64(16)).astype(np.uint16)
