"""Model-level CPU oracle: the reference's decode-session forward restated on top of
the oracle ops (liboracle.so), for end-to-end parity of small synthetic models.

TEST INFRASTRUCTURE ONLY (tests/ import it as the checker; the product never does).

Follows src/qwen_runtime.cpp: embedding row gather (:576-600), first input norm
(:602-606), layer blocks (:421-544: mixer, residual + post norm, gate/up, SwiGLU,
down, residual + next layer's input norm), LM head + argmax over the tokenizer
vocabulary (:635-639), and the MTP proposal (:715-867).  Activations are A4G128
(ActivationMode::int4, :111-128): every projection quantizes its fp16 input, takes
the exact per-group integer partials and the per-group fp32 epilogue.
Weights are the synthetic checkpoint of gfxinfer_model_create_synthetic, regenerated
with oracle.synthetic_values and quantized with the restated quantize_group128.
The layer wiring (norms, residual adds, attention gate, partial rotary, GQA grouping,
the GDN conv / decay / beta / delta rule / gated norm, final norm and head) is pinned
against HF transformers' Qwen3.5 text model with the same weights and float
projections (tests/test_oracle_model_hf.py), with planted wiring mistakes shown to fail.
"""
from __future__ import annotations

import ctypes

import numpy as np

from . import oracle as O

EPS = ctypes.c_float(1e-6)


def _laws(name: str):
    if name.endswith("conv1d.weight") or name.endswith("A_log") or name.endswith("dt_bias"):
        return 0.0, 0.5
    if name.endswith("linear_attn.norm.weight"):
        return 1.0, 0.02
    return 0.0, 0.02


class Matrix:
    """A W3/W4 projection.  `splits` selects the order of the fp32 epilogue over K: None is
    the reference's sequential epilogue (lowbit_gemv.hip:540-551); an integer S is the
    canonical order of the gfx950 library (S split-K planes, each cut into ranges of about
    ten groups, orc_gemm_epilogue_ranges), with the planes added in plane order as the
    library's residual norm adds them.  The epilogue order is the one place where the
    library's GEMMs differ from the reference's, within the fp32 tolerance."""

    def __init__(self, seed, name, fmt, rows, cols, splits=None):
        w = O.synthetic_values_c(seed, name, rows * cols, 0.02, 0.0).reshape(rows, cols)
        status, codes, scales = O.quantize_group128(w, fmt)
        assert status == 0
        del w
        self.w = O.unpack_weights(codes, rows, cols, fmt)
        self.ws16 = O.f32_to_f16_bits(scales)
        self.rows, self.cols = rows, cols
        self.splits = splits

    def __call__(self, x16: np.ndarray) -> np.ndarray:
        """fp16 [B, K] -> fp32 [B, N] through A4 activations (lowbit_gemv.hip:373-553)."""
        packed, as16 = O.quantize_activation_i4(x16)
        return self.apply(packed, as16)

    def apply(self, packed: np.ndarray, as16: np.ndarray) -> np.ndarray:
        """A4 codes [B, K/2] + fp16 scales [B, K/128] -> fp32 [B, N]."""
        a = O.unpack_a4(np.ascontiguousarray(packed), self.cols)
        partials = O.gemm_partials(self.w, a)
        if self.splits is None:
            return O.gemm_epilogue(partials, self.ws16, as16)
        planes = O.gemm_epilogue_ranges(partials, self.ws16, as16, self.splits)
        out = planes[0].copy()
        for plane in planes[1:]:
            out = (out + plane).astype(np.float32)
        return out

    def head(self, rows: int) -> "Matrix":
        m = Matrix.__new__(Matrix)
        m.w, m.ws16, m.rows, m.cols, m.splits = self.w[:rows], self.ws16[:rows], rows, self.cols, self.splits
        return m


class OracleModel:
    """The synthetic checkpoint on the CPU.  k_order: None for the reference's GEMM
    epilogue everywhere; or a function (rows, columns) -> split count, to add the group
    partials in the gfx950 library's canonical order (the residual-feeding [hidden, K]
    projections as that many split-K planes, every other projection as one).  The MTP
    weights are built on first use."""

    def __init__(self, spec: dict, seed: int, k_order=None):
        self.s = s = dict(spec)
        self.seed = seed
        self.k_order = k_order
        H, I, hd = s["hidden_size"], s["intermediate_size"], s["attention_head_size"]
        self.hd = hd
        self.q_rows = 2 * s["attention_head_count"] * hd
        self.kv_rows = s["kv_head_count"] * hd
        self.gk = s["gdn_key_head_count"] * s["gdn_head_size"]
        self.gv = s["gdn_value_head_count"] * s["gdn_head_size"]
        self.C = 2 * self.gk + self.gv

        mat, vec = self._mat, self._vec

        V = s["vocabulary_size"]
        self.embed = mat("model.language_model.embed_tokens.weight", O.W4, V, H)
        self.final_norm = vec("model.language_model.norm.weight", H)
        self.lm_head = mat("lm_head.weight", O.W4, V, H)
        self.layers = []
        for i in range(s["layer_count"]):
            p = f"model.language_model.layers.{i}."
            fmt = O.W3 if i < s["w3_mlp_layers"] else O.W4
            L = dict(attention=(i + 1) % s["full_attention_interval"] == 0,
                     input_norm=vec(p + "input_layernorm.weight", H),
                     post_norm=vec(p + "post_attention_layernorm.weight", H),
                     gate=mat(p + "mlp.gate_proj.weight", fmt, I, H),
                     up=mat(p + "mlp.up_proj.weight", fmt, I, H),
                     down=mat(p + "mlp.down_proj.weight", fmt, H, I, planes=True))
            if L["attention"]:
                self._attention(L, p)
            else:
                L.update(qkv=mat(p + "linear_attn.in_proj_qkv.weight", O.W4, self.C, H),
                         z=mat(p + "linear_attn.in_proj_z.weight", O.W4, self.gv, H),
                         a=mat(p + "linear_attn.in_proj_a.weight", O.W4, s["gdn_value_head_count"], H),
                         b=mat(p + "linear_attn.in_proj_b.weight", O.W4, s["gdn_value_head_count"], H),
                         conv=vec(p + "linear_attn.conv1d.weight", self.C * 4),
                         a_log=vec(p + "linear_attn.A_log", s["gdn_value_head_count"]),
                         dt_bias=vec(p + "linear_attn.dt_bias", s["gdn_value_head_count"]),
                         gdn_norm=vec(p + "linear_attn.norm.weight", s["gdn_head_size"]),
                         out=mat(p + "linear_attn.out_proj.weight", O.W4, H, self.gv, planes=True))
            self.layers.append(L)
        self._mtp = None

    def _mat(self, name, fmt, rows, cols, planes=False):
        splits = None
        if self.k_order is not None:
            splits = self.k_order(rows, cols) if planes else 1
        return Matrix(self.seed, name, fmt, rows, cols, splits)

    def _vec(self, name, n):
        mean, sigma = _laws(name)
        return O.f32_to_bf16_bits(O.synthetic_values(self.seed, name, n, sigma, mean))

    @property
    def mtp(self):
        """The MTP block's weights (qwen_runtime.cpp:972-1008), built on first use."""
        if self._mtp is None:
            s, mat, vec = self.s, self._mat, self._vec
            H, I = s["hidden_size"], s["intermediate_size"]
            self.mtp_fc = mat("mtp.fc.weight", O.W4, H, 2 * H)
            self.mtp_pre_embedding_norm = vec("mtp.pre_fc_norm_embedding.weight", H)
            self.mtp_pre_hidden_norm = vec("mtp.pre_fc_norm_hidden.weight", H)
            self.mtp_final_norm = vec("mtp.norm.weight", H)
            mtp = dict(attention=True, input_norm=vec("mtp.layers.0.input_layernorm.weight", H),
                       post_norm=vec("mtp.layers.0.post_attention_layernorm.weight", H),
                       gate=mat("mtp.layers.0.mlp.gate_proj.weight", O.W4, I, H),
                       up=mat("mtp.layers.0.mlp.up_proj.weight", O.W4, I, H),
                       down=mat("mtp.layers.0.mlp.down_proj.weight", O.W4, H, I, planes=True))
            self._attention(mtp, "mtp.layers.0.")
            self.draft_head = self.lm_head.head(s["mtp_draft_vocabulary"])
            self._mtp = mtp
        return self._mtp

    def _attention(self, L, p):
        s, H, hd = self.s, self.s["hidden_size"], self.hd
        mat = self._mat
        L.update(q=mat(p + "self_attn.q_proj.weight", O.W4, self.q_rows, H),
                 k=mat(p + "self_attn.k_proj.weight", O.W4, self.kv_rows, H),
                 v=mat(p + "self_attn.v_proj.weight", O.W4, self.kv_rows, H),
                 q_norm=O.f32_to_bf16_bits(O.synthetic_values(self.seed, p + "self_attn.q_norm.weight", hd, 0.02, 0.0)),
                 k_norm=O.f32_to_bf16_bits(O.synthetic_values(self.seed, p + "self_attn.k_norm.weight", hd, 0.02, 0.0)),
                 o=mat(p + "self_attn.o_proj.weight", O.W4, H, s["attention_head_count"] * hd, planes=True))


def _p(a):
    return O.ptr(np.ascontiguousarray(a))


class OracleSession:
    """Decode state of one sequence: conv/GDN states, K/V caches, positions."""

    def __init__(self, model: OracleModel, capacity: int):
        self.m = m = model
        s = m.s
        self.capacity = capacity
        gdn_layers = sum(1 for L in m.layers if not L["attention"])
        attn_layers = len(m.layers) - gdn_layers
        Hv, d = s["gdn_value_head_count"], s["gdn_head_size"]
        self.conv = [np.zeros((m.C, 4), np.uint16) for _ in range(gdn_layers)]
        self.state = [np.zeros((Hv, d, d), np.float32) for _ in range(gdn_layers)]
        self.kcache = [np.zeros((capacity, m.kv_rows), np.uint16) for _ in range(attn_layers)]
        self.vcache = [np.zeros((capacity, m.kv_rows), np.uint16) for _ in range(attn_layers)]
        self.mtp_k = np.zeros((capacity, m.kv_rows), np.uint16)
        self.mtp_v = np.zeros((capacity, m.kv_rows), np.uint16)
        self.position = 0
        self.last_hidden = None

    # ---- pieces ------------------------------------------------------------------
    def _norm(self, x16, w):
        out = np.empty_like(x16)
        O.lib().orc_rms_norm(_p(x16), _p(w), O.ptr(out), x16.shape[1], x16.shape[0], EPS, 1)
        return out

    def _residual_norm(self, res16, upd, w):
        r = np.empty_like(res16)
        n = np.empty_like(res16)
        O.lib().orc_residual_add_rms_norm(_p(res16), _p(upd), O.ptr(r), _p(w), O.ptr(n), res16.shape[1],
                                          res16.shape[0], EPS, 1)
        return r, n

    def _attention_mixer(self, L, normed, kcache, vcache, position, stop_after_append=False, raw=False):
        m, s = self.m, self.m.s
        T, hd = normed.shape[0], m.hd
        q = L["q"](normed)
        k = L["k"](normed)
        v = L["v"](normed)
        qn = np.empty((T, s["attention_head_count"], hd), np.uint16)
        kn = np.empty((T, s["kv_head_count"], hd), np.uint16)
        theta = ctypes.c_float(s["rope_theta"])
        O.lib().orc_head_norm_rope(_p(q), 2 * hd, _p(L["q_norm"]), O.ptr(qn), s["attention_head_count"], hd,
                                   s["rotary_size"], ctypes.c_uint64(position), T, theta)
        O.lib().orc_head_norm_rope(_p(k), hd, _p(L["k_norm"]), O.ptr(kn), s["kv_head_count"], hd,
                                   s["rotary_size"], ctypes.c_uint64(position), T, theta)
        O.lib().orc_kv_append(O.ptr(kn), _p(v), O.ptr(kcache), O.ptr(vcache), position, m.kv_rows, T)
        if stop_after_append:
            return None
        out = np.empty((T, s["attention_head_count"], hd), np.uint16)
        O.lib().orc_gated_attention(O.ptr(qn), _p(q), O.ptr(kcache), O.ptr(vcache), O.ptr(out), position + 1, T,
                                    s["attention_head_count"], s["kv_head_count"], hd,
                                    ctypes.c_float(np.float32(1.0 / np.sqrt(hd))))
        if raw:
            return out.reshape(T, -1)
        return L["o"](out.reshape(T, -1))

    def _gdn_mixer(self, L, normed, index, raw=False):
        m, s = self.m, self.m.s
        T = normed.shape[0]
        proj = L["qkv"](normed)
        z, a, b = L["z"](normed), L["a"](normed), L["b"](normed)
        conv_out = np.empty((T, m.C), np.uint16)
        final = np.empty_like(self.conv[index])
        O.lib().orc_gdn_conv_update(_p(proj), _p(L["conv"]), O.ptr(self.conv[index]), O.ptr(final),
                                    O.ptr(conv_out), None, m.C, T)
        self.conv[index] = final
        state = np.empty_like(self.state[index])
        out = np.empty((T, m.gv), np.uint16)
        O.lib().orc_gdn_recurrent(O.ptr(conv_out), _p(z), _p(a), _p(b), _p(L["a_log"]), _p(L["dt_bias"]),
                                  _p(L["gdn_norm"]), O.ptr(self.state[index]), O.ptr(state), O.ptr(out), None,
                                  None, None, T, s["gdn_key_head_count"], s["gdn_value_head_count"],
                                  s["gdn_head_size"])
        self.state[index] = state
        if raw:
            return out
        return L["out"](out)

    def _mlp(self, L, residual, mixer_update, next_norm):
        post, post_normed = self._residual_norm(residual, mixer_update, L["post_norm"])
        gate, up = L["gate"](post_normed), L["up"](post_normed)
        act = np.empty(gate.shape, np.uint16)
        O.lib().orc_silu_multiply(_p(gate), _p(up), O.ptr(act), gate.size)
        return self._residual_norm(post, L["down"](act), next_norm)

    # ---- one layer, teacher-forced (qwen_runtime.cpp:421-544) ----------------------
    def layer_forward(self, i: int, residual16: np.ndarray, position: int) -> np.ndarray:
        """Layer i of a block whose residual rows entering the layer are `residual16`
        (fp16 [T, H], e.g. another implementation's), from this session's state of that
        layer (which it advances); returns the residual rows leaving the layer."""
        m = self.m
        L = m.layers[i]
        normed = self._norm(residual16, L["input_norm"])
        index = sum(1 for M in m.layers[:i] if M["attention"] == L["attention"])
        if L["attention"]:
            update = self._attention_mixer(L, normed, self.kcache[index], self.vcache[index], position)
        else:
            update = self._gdn_mixer(L, normed, index)
        hidden, _ = self._mlp(L, residual16, update, L["input_norm"])
        return hidden

    # ---- one layer, stage by stage, each stage from given inputs -------------------
    def _index(self, i):
        L = self.m.layers[i]
        return L, sum(1 for M in self.m.layers[:i] if M["attention"] == L["attention"])

    def mixer_stage(self, i, residual16, position):
        """Input norm + mixer of layer i up to its fp16 output, as A4 codes and scales (the
        o / out projection's input); advances this session's state of the layer."""
        L, index = self._index(i)
        normed = self._norm(residual16, L["input_norm"])
        if L["attention"]:
            out = self._attention_mixer(L, normed, self.kcache[index], self.vcache[index], position, raw=True)
        else:
            out = self._gdn_mixer(L, normed, index, raw=True)
        return O.quantize_activation_i4(out)

    def post_stage(self, i, residual16, mixer_codes, mixer_scales):
        """o / out projection of given A4 codes + residual add: the rows after the mixer."""
        L, _ = self._index(i)
        update = (L["o"] if L["attention"] else L["out"]).apply(mixer_codes, mixer_scales)
        post, _ = self._residual_norm(residual16, update, L["post_norm"])
        return post

    def mlp_codes_stage(self, i, post16):
        """Post norm, gate/up, SwiGLU: the down projection's A4 codes and scales."""
        L, _ = self._index(i)
        normed = self._norm(post16, L["post_norm"])
        gate, up = L["gate"](normed), L["up"](normed)
        act = np.empty(gate.shape, np.uint16)
        O.lib().orc_silu_multiply(_p(gate), _p(up), O.ptr(act), gate.size)
        return O.quantize_activation_i4(act)

    def out_stage(self, i, post16, mlp_codes, mlp_scales):
        """Down projection of given A4 codes + residual add: the rows leaving the layer."""
        L, _ = self._index(i)
        hidden, _ = self._residual_norm(post16, L["down"].apply(mlp_codes, mlp_scales), L["post_norm"])
        return hidden

    def final_logits(self, residual16: np.ndarray) -> np.ndarray:
        """Final norm + LM head of residual rows leaving the last layer (qwen_runtime.cpp:635)."""
        return self.m.lm_head(self._norm(residual16, self.m.final_norm))

    # ---- QwenDecodeSession::block_step (qwen_runtime.cpp:1320-1392) --------------
    def block_step(self, tokens):
        m, s = self.m, self.m.s
        T = len(tokens)
        hidden = np.stack([self._gather(t) for t in tokens])
        normed = self._norm(hidden, m.layers[0]["input_norm"])
        gdn_i = attn_i = 0
        for i, L in enumerate(m.layers):
            next_norm = m.layers[i + 1]["input_norm"] if i + 1 < len(m.layers) else m.final_norm
            if L["attention"]:
                update = self._attention_mixer(L, normed, self.kcache[attn_i], self.vcache[attn_i], self.position)
                attn_i += 1
            else:
                update = self._gdn_mixer(L, normed, gdn_i)
                gdn_i += 1
            hidden, normed = self._mlp(L, hidden, update, next_norm)
        logits = m.lm_head(normed)
        out = np.empty(T, np.uint32)
        O.lib().orc_argmax(O.ptr(logits), s["tokenizer_vocabulary_size"], s["vocabulary_size"], T, None,
                           O.ptr(out))
        self.position += T
        self.last_hidden = hidden[-1:].copy()
        return [int(x) for x in out], logits

    def _gather(self, token):
        """launch_lowbit_row_gather: fp16(w(row, c) * ws(row, c/128)) (lowbit_gemv.hip:191-231)."""
        m = self.m.embed
        scales = O.f16_bits_to_f32(m.ws16[token]).repeat(128)
        return O.f32_to_f16_bits(m.w[token].astype(np.float32) * scales)

    # ---- launch_mtp_proposal (qwen_runtime.cpp:715-867) ---------------------------
    def mtp_proposal(self, token, conditioning16, position):
        m, s = self.m, self.m.s
        H = s["hidden_size"]
        m.mtp  # builds the MTP weights on first use
        emb = self._gather(token)[None, :]
        concat = np.empty((1, 2 * H), np.uint16)
        O.lib().orc_dual_rms_norm_concat(O.ptr(emb), _p(m.mtp_pre_embedding_norm), _p(conditioning16),
                                         _p(m.mtp_pre_hidden_norm), O.ptr(concat), H, EPS, 1)
        fc = m.mtp_fc(concat)
        mtp_input = O.f32_to_f16_bits(fc)                  # launch_gfx12_i4_gemm_half
        normed = self._norm(mtp_input, m.mtp["input_norm"])
        update = self._attention_mixer(m.mtp, normed, self.mtp_k, self.mtp_v, position)
        hidden, normed = self._mlp(m.mtp, mtp_input, update, m.mtp_final_norm)
        logits = m.draft_head(normed)
        out = np.empty(1, np.uint32)
        O.lib().orc_argmax(O.ptr(logits), s["mtp_draft_vocabulary"], s["mtp_draft_vocabulary"], 1, None,
                           O.ptr(out))
        return int(out[0]), logits, hidden
