"""Python view of the decode runtime (include/gfxinfer_runtime.h).

`SyntheticModel` stands where the reference's `gfxinfer::Engine` stands
(include/gfxinfer/engine.h), holding a seeded synthetic checkpoint in the gfx950
tile layout; `QwenDecodeSession` mirrors `gfxinfer::QwenDecodeSession`
(include/gfxinfer/qwen_runtime.h:47-77) method for method: greedy_step,
block_step, mtp_draft, speculative_step, position, summary.  Errors raise
GfxinferError with the reference ErrorCode value.  All work runs in
libgfxinfer_amd.so; this module only marshals arguments.
"""
from __future__ import annotations

import atexit
import ctypes
import weakref
from dataclasses import dataclass

import numpy as np

from . import GfxinferError, check, lib

U32 = ctypes.c_uint32

# Handles still open at interpreter exit are closed by atexit (sessions before the
# models they use), while the HIP runtime is intact: a destructor run during the
# interpreter's final teardown would call into an already-finalized runtime.
_LIVE_SESSIONS: "weakref.WeakSet" = weakref.WeakSet()
_LIVE_OTHERS: "weakref.WeakSet" = weakref.WeakSet()


@atexit.register
def _close_live_handles() -> None:
    for group in (_LIVE_SESSIONS, _LIVE_OTHERS):
        for obj in list(group):
            try:
                obj.close()
            except Exception:
                pass


class ModelSpec(ctypes.Structure):
    """gfxinfer_model_spec (qwen38_spec.h:15-48 as fields)."""
    _fields_ = [(name, ctypes.c_uint32) for name in (
        "hidden_size", "intermediate_size", "layer_count", "full_attention_interval",
        "attention_head_count", "kv_head_count", "attention_head_size", "rotary_size",
        "gdn_key_head_count", "gdn_value_head_count", "gdn_head_size", "vocabulary_size",
        "tokenizer_vocabulary_size", "mtp_draft_vocabulary", "w3_mlp_layers")] + [
        ("rms_norm_epsilon", ctypes.c_float), ("rope_theta", ctypes.c_float)]

    def as_dict(self) -> dict:
        return {name: getattr(self, name) for name, _ in self._fields_}


def qwen38_27b_spec() -> ModelSpec:
    spec = ModelSpec()
    lib().gfxinfer_model_spec_qwen38_27b(ctypes.byref(spec))
    return spec


def qwen38_reference_spec() -> ModelSpec:
    """The reference's own Qwen3.8 shape (24/4 x 256 attention, 16/48 GDN heads)."""
    spec = ModelSpec()
    lib().gfxinfer_model_spec_qwen38_reference(ctypes.byref(spec))
    return spec


def tiny_spec(**overrides) -> ModelSpec:
    """A small model of the same structure for oracle parity (2 GDN + 2 attention layers)."""
    spec = qwen38_27b_spec()
    values = dict(hidden_size=256, intermediate_size=512, layer_count=4, attention_head_count=4,
                  kv_head_count=2, rotary_size=64, gdn_key_head_count=2, gdn_value_head_count=16,
                  vocabulary_size=1024, tokenizer_vocabulary_size=1000, mtp_draft_vocabulary=512,
                  w3_mlp_layers=2)
    values.update(overrides)
    for k, v in values.items():
        setattr(spec, k, v)
    return spec


class SpecTensor(ctypes.Structure):
    """gfxinfer_spec_tensor: one entry of a spec's tensor table (converter naming)."""
    _fields_ = [("name", ctypes.c_char * 96), ("format", ctypes.c_int32), ("rows", ctypes.c_uint64),
                ("columns", ctypes.c_uint64), ("mean", ctypes.c_float), ("sigma", ctypes.c_float)]


def spec_tensors(spec: ModelSpec) -> list[dict]:
    """The tensors a model of `spec` binds (host only): name, format, rows, columns and
    the synthetic value law."""
    out = []
    for i in range(int(lib().gfxinfer_model_spec_tensor_count(ctypes.byref(spec)))):
        t = SpecTensor()
        check(lib().gfxinfer_model_spec_tensor(ctypes.byref(spec), i, ctypes.byref(t)))
        out.append(dict(name=t.name.decode(), format=int(t.format), rows=int(t.rows), columns=int(t.columns),
                        mean=float(t.mean), sigma=float(t.sigma)))
    return out


def artifact_tiny_spec() -> ModelSpec:
    """The smallest spec the kernels accept (one GDN and one attention layer, hidden 128),
    used for the committed gfx1200 artifact fixture."""
    return tiny_spec(hidden_size=128, intermediate_size=128, layer_count=2, full_attention_interval=2,
                     attention_head_count=1, kv_head_count=1, gdn_key_head_count=1, gdn_value_head_count=16,
                     vocabulary_size=256, tokenizer_vocabulary_size=250, mtp_draft_vocabulary=128,
                     w3_mlp_layers=1)


def reference_tiny_spec(**overrides) -> ModelSpec:
    """A small model of the reference's own head shapes (qwen38_spec.h:22-29): attention
    heads of 256 dims with six query heads per KV head and rotary 64, GDN 16 key / 48
    value heads (three value heads per key head, 10240 conv channels)."""
    values = dict(attention_head_count=6, kv_head_count=1, attention_head_size=256, rotary_size=64,
                  gdn_key_head_count=16, gdn_value_head_count=48, full_attention_interval=2)
    values.update(overrides)
    return tiny_spec(**values)


def artifact_reference_tiny_spec() -> ModelSpec:
    """reference_tiny_spec() at the smallest widths (one GDN and one attention layer,
    hidden 128), used for the committed gfx1200 artifact of the reference's shape."""
    return reference_tiny_spec(hidden_size=128, intermediate_size=256, layer_count=2, vocabulary_size=256,
                               tokenizer_vocabulary_size=250, mtp_draft_vocabulary=128, w3_mlp_layers=1)


class TensorView(ctypes.Structure):
    """gfxinfer_tensor_view (engine.h:47-60 DeviceTensorView)."""
    _fields_ = [("format", ctypes.c_int32), ("rows", ctypes.c_uint64), ("columns", ctypes.c_uint64),
                ("data", ctypes.c_void_p), ("auxiliary", ctypes.c_void_p),
                ("data_bytes", ctypes.c_size_t), ("auxiliary_bytes", ctypes.c_size_t)]


class SessionConfig(ctypes.Structure):
    """gfxinfer_session_config (qwen_runtime.h:23-29 DecodeSessionConfig)."""
    _fields_ = [("maximum_context_tokens", ctypes.c_size_t), ("graph_verifier_batch", ctypes.c_uint32),
                ("keep_logits", ctypes.c_int32)]


class SessionSummary(ctypes.Structure):
    """gfxinfer_session_summary (qwen_runtime.h:31-37)."""
    _fields_ = [(name, ctypes.c_size_t) for name in (
        "arena_bytes", "maximum_context_tokens", "gdn_state_bytes", "kv_cache_bytes", "mtp_cache_bytes")]


class SpeculativeResult(ctypes.Structure):
    """gfxinfer_speculative_result (qwen_runtime.h:39-45 SpeculativeStepResult)."""
    _fields_ = [("tokens", ctypes.c_uint32 * 32), ("token_count", ctypes.c_uint32),
                ("proposed_drafts", ctypes.c_uint32), ("accepted_drafts", ctypes.c_uint32)]


@dataclass
class SpeculativeStepResult:
    tokens: list[int]
    proposed_drafts: int
    accepted_drafts: int


class GenerateConfig(ctypes.Structure):
    _fields_ = [("maximum_tokens", ctypes.c_uint32), ("draft_count", ctypes.c_uint32),
                ("adaptive_depth", ctypes.c_int32), ("stop_tokens", ctypes.c_void_p),
                ("stop_count", ctypes.c_uint32)]


class GenerateStats(ctypes.Structure):
    _fields_ = [("prompt_tokens", ctypes.c_size_t), ("output_tokens", ctypes.c_size_t),
                ("speculative_rounds", ctypes.c_size_t), ("proposed_drafts", ctypes.c_size_t),
                ("accepted_drafts", ctypes.c_size_t), ("speculative_emitted", ctypes.c_size_t),
                ("prefill_ms", ctypes.c_double), ("decode_ms", ctypes.c_double)]

    def as_dict(self) -> dict:
        return {name: getattr(self, name) for name, _ in self._fields_}


class DepthPolicy:
    """Online MTP depth selection (gfxinfer_depth_policy_*)."""

    def __init__(self, maximum_depth: int):
        handle = ctypes.c_void_p()
        check(lib().gfxinfer_depth_policy_create(maximum_depth, ctypes.byref(handle)))
        self._handle = handle
        _LIVE_OTHERS.add(self)

    def choose(self, limit: int) -> int:
        return int(lib().gfxinfer_depth_policy_choose(self._handle, limit))

    def record(self, depth: int, emitted: int, milliseconds: float) -> None:
        check(lib().gfxinfer_depth_policy_record(self._handle, depth, emitted, milliseconds))

    def close(self):
        if self._handle is not None:
            lib().gfxinfer_depth_policy_destroy(self._handle)
            self._handle = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


class ArtifactIdentity(ctypes.Structure):
    """gfxinfer_artifact_identity (artifact.h:35-40 ArtifactIdentity)."""
    _fields_ = [("target_arch", ctypes.c_char * 16), ("model_id", ctypes.c_char * 32),
                ("weights_id", ctypes.c_char * 32), ("recipe_id", ctypes.c_char * 64)]


class ArtifactTensor(ctypes.Structure):
    """gfxinfer_artifact_tensor (artifact.h:42-55 TensorDescriptor)."""
    _fields_ = [("name", ctypes.c_char_p), ("dtype", ctypes.c_uint16), ("quantization", ctypes.c_uint16),
                ("rank", ctypes.c_uint16), ("flags", ctypes.c_uint16), ("alignment", ctypes.c_uint32),
                ("dimensions", ctypes.c_uint64 * 4), ("data_offset", ctypes.c_uint64),
                ("data_bytes", ctypes.c_uint64), ("aux_offset", ctypes.c_uint64),
                ("aux_bytes", ctypes.c_uint64), ("data_crc64", ctypes.c_uint64)]

    @property
    def shape(self) -> tuple:
        return tuple(int(self.dimensions[i]) for i in range(self.rank))


class Artifact:
    """A mapped, validated .gfxi file (ArtifactView, artifact.h:81-120)."""

    def __init__(self, path: str, verify_checksums: bool = True):
        handle = ctypes.c_void_p()
        check(lib().gfxinfer_artifact_open(str(path).encode(), int(verify_checksums), ctypes.byref(handle)))
        self._handle = handle

    def close(self):
        if self._handle is not None:
            lib().gfxinfer_artifact_close(self._handle)
            self._handle = None

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def identity(self) -> dict:
        ident = ArtifactIdentity()
        check(lib().gfxinfer_artifact_get_identity(self._handle, ctypes.byref(ident)))
        return {k: getattr(ident, k).decode() for k in ("target_arch", "model_id", "weights_id", "recipe_id")}

    def tensors(self) -> list:
        out = []
        for i in range(int(lib().gfxinfer_artifact_tensor_count(self._handle))):
            t = ArtifactTensor()
            check(lib().gfxinfer_artifact_tensor_at(self._handle, i, ctypes.byref(t)))
            out.append(t)
        return out

    def find(self, name: str) -> ArtifactTensor:
        t = ArtifactTensor()
        check(lib().gfxinfer_artifact_find(self._handle, name.encode(), ctypes.byref(t)))
        return t

    def resource(self, name: str) -> bytes:
        """Engine::resource (engine.cpp:229-236): an unquantized u8 "resources/..." tensor."""
        data = ctypes.c_void_p()
        n = ctypes.c_uint64()
        check(lib().gfxinfer_artifact_resource(self._handle, name.encode(), ctypes.byref(data), ctypes.byref(n)))
        return ctypes.string_at(data.value, n.value) if n.value else b""

    def payload(self, t: ArtifactTensor, auxiliary: bool = False) -> np.ndarray:
        offset, n = (t.aux_offset, t.aux_bytes) if auxiliary else (t.data_offset, t.data_bytes)
        ptr = lib().gfxinfer_artifact_bytes(self._handle, offset, n)
        if ptr is None:
            raise GfxinferError(1, "payload outside the artifact")
        return np.frombuffer((ctypes.c_uint8 * n).from_address(ptr), np.uint8).copy()


class Tokenizer:
    """Byte-level BPE of a tokenizer.json document (QwenTokenizer, tokenizer.h:17-32):
    from_json / encode / decode / vocabulary_size, run by libgfxinfer_amd.so."""

    def __init__(self, tokenizer_json: bytes):
        data = bytes(tokenizer_json)
        handle = ctypes.c_void_p()
        buf = ctypes.create_string_buffer(data, len(data)) if data else None
        check(lib().gfxinfer_tokenizer_create(buf, len(data), ctypes.byref(handle)))
        self._handle = handle
        _LIVE_OTHERS.add(self)

    @classmethod
    def from_file(cls, path: str) -> "Tokenizer":
        with open(path, "rb") as f:
            return cls(f.read())

    def close(self):
        if getattr(self, "_handle", None) is not None:
            lib().gfxinfer_tokenizer_destroy(self._handle)
            self._handle = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    @property
    def vocabulary_size(self) -> int:
        return int(lib().gfxinfer_tokenizer_vocabulary_size(self._handle))

    def encode(self, text: str) -> list[int]:
        raw = text.encode("utf-8")
        count = ctypes.c_size_t()
        capacity = len(raw) + 16  # at most one id per byte, plus added tokens
        ids = np.empty(capacity, np.uint32)
        check(lib().gfxinfer_tokenizer_encode(self._handle, raw, len(raw), ids.ctypes.data, capacity,
                                              ctypes.byref(count)))
        if count.value > capacity:
            ids = np.empty(count.value, np.uint32)
            check(lib().gfxinfer_tokenizer_encode(self._handle, raw, len(raw), ids.ctypes.data, count.value,
                                                  ctypes.byref(count)))
        return [int(i) for i in ids[:count.value]]

    def decode_bytes(self, ids) -> bytes:
        arr = np.ascontiguousarray(np.asarray(list(ids), dtype=np.int64).astype(np.uint32))
        length = ctypes.c_size_t()
        check(lib().gfxinfer_tokenizer_decode(self._handle, arr.ctypes.data if arr.size else None, arr.size,
                                              None, 0, ctypes.byref(length)))
        out = ctypes.create_string_buffer(max(length.value, 1))
        check(lib().gfxinfer_tokenizer_decode(self._handle, arr.ctypes.data if arr.size else None, arr.size,
                                              out, length.value, ctypes.byref(length)))
        return out.raw[:length.value]

    def decode(self, ids) -> str:
        return self.decode_bytes(ids).decode("utf-8", errors="replace")


def render_chat_prompt(prompt: str) -> str:
    """The generate command's chat rendering (cli/main.cpp:1037-1039)."""
    raw = prompt.encode("utf-8")
    length = ctypes.c_size_t()
    check(lib().gfxinfer_render_chat_prompt(raw, len(raw), None, 0, ctypes.byref(length)))
    out = ctypes.create_string_buffer(length.value)
    check(lib().gfxinfer_render_chat_prompt(raw, len(raw), out, length.value, ctypes.byref(length)))
    return out.raw[:length.value].decode("utf-8")


# The chat special tokens that end a generated answer (cli/main.cpp:1100-1103 stops at
# the ids of <|im_end|> and <|endoftext|> of the model's own tokenizer).
STOP_PIECES = ("<|im_end|>", "<|endoftext|>")


def generate_text(session: "QwenDecodeSession", tokenizer: Tokenizer, prompt: str, maximum_tokens: int,
                  draft_count: int = 0, adaptive_depth: bool = False) -> dict:
    """The generate command's text path (cli/main.cpp:1023-1120) over the session API:
    render the one-turn chat prompt, encode it, run the generate loop (prefill, then
    greedy or speculative rounds) until `maximum_tokens` or a stop token, decode the
    generated ids.  Returns the prompt ids, the generated ids, their decoded bytes and
    the loop statistics; raises GfxinferError when the prompt and the generation do
    not fit the session's context, as the command refuses to run."""
    ids = tokenizer.encode(render_chat_prompt(prompt))
    stops = []
    for piece in STOP_PIECES:
        encoded = tokenizer.encode(piece)
        if len(encoded) == 1:
            stops.append(encoded[0])
    tokens, stats = session.generate(ids, maximum_tokens, draft_count, adaptive_depth, stops)
    return {"prompt_ids": ids, "tokens": tokens, "text": tokenizer.decode_bytes(tokens), "stats": stats,
            "stop_ids": stops}


def crc64_ecma(data: bytes, state: int = 0) -> int:
    """CRC-64/ECMA-182 (artifact.cpp:187-213)."""
    buf = np.frombuffer(bytes(data), np.uint8)
    return int(lib().gfxinfer_crc64_ecma(state, buf.ctypes.data if len(buf) else None, len(buf)))


def retile_gfx12_for_gfx950(fmt: int, gfx12_codes: np.ndarray) -> np.ndarray:
    src = np.ascontiguousarray(gfx12_codes, np.uint8)
    out = np.empty_like(src)
    check(lib().gfxinfer_retile_gfx12_for_gfx950(fmt, src.ctypes.data, src.nbytes, out.ctypes.data))
    return out


class SyntheticModel:
    """Seeded synthetic checkpoint on one device (Engine::create equivalent), or, with
    from_artifact(), the weights of a .gfxi artifact."""

    def __init__(self, spec: ModelSpec, seed: int, device: int = 0):
        self.spec = spec
        self.seed = seed
        handle = ctypes.c_void_p()
        check(lib().gfxinfer_model_create_synthetic(ctypes.byref(spec), seed, device, ctypes.byref(handle)))
        self._handle = handle
        _LIVE_OTHERS.add(self)

    @classmethod
    def from_artifact(cls, spec: ModelSpec, path: str, verify_checksums: bool = True, device: int = 0):
        self = cls.__new__(cls)
        self.spec = spec
        self.seed = None
        handle = ctypes.c_void_p()
        check(lib().gfxinfer_model_create_from_artifact(ctypes.byref(spec), str(path).encode(),
                                                        int(verify_checksums), device, ctypes.byref(handle)))
        self._handle = handle
        _LIVE_OTHERS.add(self)
        return self

    def write_artifact(self, path: str, weights_id: str, draft_rows=None):
        rows = None if draft_rows is None else np.ascontiguousarray(draft_rows, np.uint32)
        check(lib().gfxinfer_model_write_artifact(self.handle, str(path).encode(), weights_id.encode(),
                                                  None if rows is None else rows.ctypes.data,
                                                  0 if rows is None else len(rows)))

    @property
    def handle(self):
        if self._handle is None:
            raise GfxinferError(1, "model was closed")
        return self._handle

    def close(self):
        if self._handle is not None:
            lib().gfxinfer_model_destroy(self._handle)
            self._handle = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    @property
    def weight_bytes(self) -> int:
        return int(lib().gfxinfer_model_weight_bytes(self.handle))

    @property
    def stream(self) -> int:
        return lib().gfxinfer_model_stream(self.handle)

    def find_tensor(self, name: str) -> TensorView:
        view = TensorView()
        check(lib().gfxinfer_model_find_tensor(self.handle, name.encode(), ctypes.byref(view)))
        return view

    def tensor_bytes(self, name: str, auxiliary: bool = False) -> np.ndarray:
        view = self.find_tensor(name)
        n = view.auxiliary_bytes if auxiliary else view.data_bytes
        out = np.empty(n, np.uint8)
        check(lib().gfxinfer_model_copy_tensor(self.handle, name.encode(), int(auxiliary),
                                               out.ctypes.data, n))
        return out


class QwenDecodeSession:
    """QwenDecodeSession (qwen_runtime.h:47-77) over a SyntheticModel."""

    def __init__(self, model: SyntheticModel, maximum_context_tokens: int = 4096,
                 graph_verifier_batch: int = 0, keep_logits: bool = False):
        self.model = model
        config = SessionConfig(maximum_context_tokens, graph_verifier_batch, int(keep_logits))
        handle = ctypes.c_void_p()
        check(lib().gfxinfer_session_create(model.handle, ctypes.byref(config), ctypes.byref(handle)))
        self._handle = handle
        _LIVE_SESSIONS.add(self)

    def close(self):
        if self._handle is not None:
            lib().gfxinfer_session_destroy(self._handle)
            self._handle = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def greedy_step(self, token: int) -> int:
        out = U32()
        check(lib().gfxinfer_session_greedy_step(self._handle, token, ctypes.byref(out)))
        return out.value

    def block_step(self, tokens) -> list[int]:
        arr = np.ascontiguousarray(tokens, dtype=np.uint32)
        out = np.zeros(len(arr), np.uint32)
        check(lib().gfxinfer_session_block_step(self._handle, arr.ctypes.data, len(arr), out.ctypes.data))
        return [int(x) for x in out]

    def mtp_draft(self, token: int) -> int:
        out = U32()
        check(lib().gfxinfer_session_mtp_draft(self._handle, token, ctypes.byref(out)))
        return out.value

    @staticmethod
    def _result(r: SpeculativeResult) -> SpeculativeStepResult:
        return SpeculativeStepResult([int(r.tokens[i]) for i in range(r.token_count)],
                                     int(r.proposed_drafts), int(r.accepted_drafts))

    def speculative_step(self, seed: int, draft_count: int) -> SpeculativeStepResult:
        r = SpeculativeResult()
        check(lib().gfxinfer_session_speculative_step(self._handle, seed, draft_count, ctypes.byref(r)))
        return self._result(r)

    def speculative_step_forced(self, seed: int, draft_count: int, accepted: int) -> SpeculativeStepResult:
        r = SpeculativeResult()
        check(lib().gfxinfer_session_speculative_step_forced(self._handle, seed, draft_count, accepted,
                                                             ctypes.byref(r)))
        return self._result(r)

    def speculative_step_planted(self, seed: int, drafts) -> SpeculativeStepResult:
        arr = np.ascontiguousarray(drafts, dtype=np.uint32)
        r = SpeculativeResult()
        check(lib().gfxinfer_session_speculative_step_planted(self._handle, seed, len(arr), arr.ctypes.data,
                                                              ctypes.byref(r)))
        return self._result(r)

    def prefill(self, tokens, sync_mtp: bool = True) -> int:
        """Chunked prefill; returns the greedy token after the last prompt token."""
        arr = np.ascontiguousarray(tokens, dtype=np.uint32)
        out = U32()
        check(lib().gfxinfer_session_prefill(self._handle, arr.ctypes.data, len(arr), int(sync_mtp),
                                             ctypes.byref(out)))
        return out.value

    def generate(self, prompt, maximum_tokens: int, draft_count: int = 0, adaptive_depth: bool = False,
                 stop_tokens=()):
        """The reference CLI generate loop; returns (tokens, stats dict)."""
        arr = np.ascontiguousarray(prompt, dtype=np.uint32)
        stops = np.ascontiguousarray(stop_tokens, dtype=np.uint32)
        cfg = GenerateConfig(maximum_tokens, draft_count, int(adaptive_depth),
                             stops.ctypes.data if len(stops) else None, len(stops))
        out = np.zeros(maximum_tokens, np.uint32)
        count = ctypes.c_size_t()
        stats = GenerateStats()
        check(lib().gfxinfer_session_generate(self._handle, arr.ctypes.data, len(arr), ctypes.byref(cfg),
                                              out.ctypes.data, ctypes.byref(count), ctypes.byref(stats)))
        return [int(x) for x in out[:count.value]], stats.as_dict()

    def position(self) -> int:
        return int(lib().gfxinfer_session_position(self._handle))

    def mtp_position(self) -> int:
        return int(lib().gfxinfer_session_mtp_position(self._handle))

    def summary(self) -> SessionSummary:
        s = SessionSummary()
        check(lib().gfxinfer_session_get_summary(self._handle, ctypes.byref(s)))
        return s

    def layer_trace_bytes(self) -> int:
        return int(lib().gfxinfer_session_layer_trace_bytes(self._handle))

    def set_layer_trace(self, device_pointer, nbytes: int) -> None:
        """Per-layer stage boundaries into a device buffer (test hook; 0 turns it off)."""
        check(lib().gfxinfer_session_set_layer_trace(self._handle, device_pointer or None, nbytes))

    def buffer(self, name: str, dtype=np.uint8, count: int | None = None, offset: int = 0) -> np.ndarray:
        """Copy of a named session buffer (test accessor)."""
        total = int(lib().gfxinfer_session_buffer_bytes(self._handle, name.encode()))
        if total == 0:
            raise GfxinferError(1, f"unknown session buffer {name}")
        itemsize = np.dtype(dtype).itemsize
        nbytes = (total - offset) if count is None else count * itemsize
        out = np.empty(nbytes // itemsize, dtype)
        check(lib().gfxinfer_session_copy_buffer(self._handle, name.encode(), offset, out.ctypes.data,
                                                 out.nbytes))
        return out
