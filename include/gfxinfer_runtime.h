/*
 * gfxinfer_amd runtime: the MTP speculative-decoding session behind a C ABI.
 *
 * Replaces the reference's C++ runtime entry points (include/gfxinfer/engine.h,
 * include/gfxinfer/qwen_runtime.h) with opaque handles and plain structs:
 *  - gfxinfer_model    ~ gfxinfer::Engine: one device arena of weights in the gfx950
 *                        tile layout plus the compute stream;
 *  - gfxinfer_session  ~ gfxinfer::QwenDecodeSession: session arena, 64-layer
 *                        verifier, MTP proposal chain, GDN rollback, hipGraphs.
 * Status codes and gfxinfer_last_error() are those of gfxinfer_amd.h.  Every
 * call runs on the model's compute stream; step calls synchronize it before they
 * return, as the reference methods do.  Handles are single-owner and not
 * thread-safe (qwen_runtime.h:47-77).
 */
#ifndef GFXINFER_RUNTIME_H
#define GFXINFER_RUNTIME_H

#include "gfxinfer_amd.h"

#ifdef __cplusplus
extern "C" {
#endif

/* Model shape.  The reference bakes these into include/gfxinfer/qwen38_spec.h:15-48
 * (Qwen38Spec); here they are fields so the same code runs the 27B-shaped model and
 * small test models. */
typedef struct gfxinfer_model_spec {
  uint32_t hidden_size;               /* qwen38_spec.h:18 */
  uint32_t intermediate_size;         /* :19 */
  uint32_t layer_count;               /* :20 */
  uint32_t full_attention_interval;   /* :21; layer i is attention iff (i+1) % interval == 0 */
  uint32_t attention_head_count;      /* :22 */
  uint32_t kv_head_count;             /* :23 */
  uint32_t attention_head_size;       /* :24; 128 or 256 */
  uint32_t rotary_size;               /* :25 */
  uint32_t gdn_key_head_count;        /* :26 */
  uint32_t gdn_value_head_count;      /* :28 */
  uint32_t gdn_head_size;             /* :27, :29; must be 128 */
  uint32_t vocabulary_size;           /* :16; LM head and embedding rows */
  uint32_t tokenizer_vocabulary_size; /* :17; argmax range of the verifier */
  uint32_t mtp_draft_vocabulary;      /* qwen_runtime.cpp:47 kMtpDraftVocabulary */
  uint32_t w3_mlp_layers;             /* converter.cpp:98-119: MLP of layers < this is W3, else W4 */
  float rms_norm_epsilon;             /* qwen38_spec.h:33 */
  float rope_theta;                   /* qwen38_spec.h:34 */
} gfxinfer_model_spec;

/* Fills the synthetic Qwen3.8-27B shape: 64 layers (48 GDN + 16 attention), hidden 5120,
 * MLP 17408 (W3 in layers 0-55, W4 in 56-63), attention 40 Q / 8 KV heads x 128 with
 * rotary 64, GDN 16 key / 32 value heads x 128, vocabulary 151936, MTP shortlist 98304. */
void gfxinfer_model_spec_qwen38_27b(gfxinfer_model_spec* spec);

/* Fills the reference's own model shape (qwen38_spec.h:16-34): as above but attention
 * 24 Q / 4 KV heads x 256 with rotary 64, GDN 16 key / 48 value heads x 128 (10240 conv
 * channels), vocabulary 248320 (tokenizer 248077); MLP in W3 except the last 8 layers
 * (converter.h:20-23 with mlp_bits 3). */
void gfxinfer_model_spec_qwen38_reference(gfxinfer_model_spec* spec);

typedef struct gfxinfer_model gfxinfer_model;

/* Engine::create (engine.h:80-86) for a synthetic checkpoint: allocates one device
 * arena, fills every tensor of the converter's naming (converter.cpp:78-119) with seeded
 * values and quantizes the 2-D ones on the device with the group-128 quantizer
 * (W3 for MLP layers < w3_mlp_layers, W4 for every other matrix; norms, conv1d,
 * A_log and dt_bias stay bf16).  Values: matrices N(0, 0.02); (1+w) norms N(0, 0.02);
 * the GDN output norm 1 + N(0, 0.02); conv1d N(0, 0.5); A_log and dt_bias N(0, 0.5).
 * The generator is a counter-based integer hash (splitmix64, Irwin-Hall of twelve
 * 16-bit uniforms), so a CPU restatement reproduces every value bit for bit. */
int32_t gfxinfer_model_create_synthetic(const gfxinfer_model_spec* spec, uint64_t seed,
                                        int32_t device, gfxinfer_model** out);
/* Releases the model.  Sessions created on it keep it alive: with sessions still open the
 * weights and stream are freed when the last of them is destroyed (a session borrows the
 * model's stream and arena).  No reference counterpart: the reference's session holds an
 * Engine& that must outlive it. */
void gfxinfer_model_destroy(gfxinfer_model* model);
/* Engine::compute_stream (engine.h:89): the hipStream_t every session call runs on. */
void* gfxinfer_model_stream(const gfxinfer_model* model);
size_t gfxinfer_model_weight_bytes(const gfxinfer_model* model);

/* DeviceTensorView (engine.h:47-60).  format: GFXI_W3G128 / GFXI_W4G128 for tiled
 * matrices (data = tiled codes, auxiliary = tiled fp16 scales), 0 for bf16 vectors
 * (data = bf16 values, auxiliary = NULL), -1 for int32 vectors (draft-head token ids). */
typedef struct gfxinfer_tensor_view {
  int32_t format;
  uint64_t rows;
  uint64_t columns;
  void* data;
  void* auxiliary;
  size_t data_bytes;
  size_t auxiliary_bytes;
} gfxinfer_tensor_view;

/* One entry of the tensor table a spec implies, in converter naming (converter.cpp:78-119):
 * format as in gfxinfer_tensor_view, shape, and the synthetic value law mean + sigma * N(0, 1).
 * Host only (no device access).  No reference counterpart: it lets a host tool (a converter
 * or a fixture writer) enumerate what gfxinfer_model_create_from_artifact binds. */
typedef struct gfxinfer_spec_tensor {
  char name[96];
  int32_t format;
  uint64_t rows;
  uint64_t columns;
  float mean;
  float sigma;
} gfxinfer_spec_tensor;
size_t gfxinfer_model_spec_tensor_count(const gfxinfer_model_spec* spec);
int32_t gfxinfer_model_spec_tensor(const gfxinfer_model_spec* spec, size_t index,
                                   gfxinfer_spec_tensor* out);

/* Engine::find_device_tensor (engine.h:87-88). */
int32_t gfxinfer_model_find_tensor(const gfxinfer_model* model, const char* name,
                                   gfxinfer_tensor_view* out);
/* Copies a tensor's data (or auxiliary, when `auxiliary` is non-zero) into host memory
 * of `bytes` bytes.  No reference counterpart: a test accessor. */
int32_t gfxinfer_model_copy_tensor(const gfxinfer_model* model, const char* name,
                                   int32_t auxiliary, void* host, size_t bytes);

/* ---- .gfxi artifacts (artifact.h, artifact.cpp; converter.cpp) --------------------
 * The reference's file format: 256-byte header, 128-byte directory entries, name table,
 * 256-byte aligned payloads, CRC-64/ECMA-182 over the manifest and every tensor's data.
 * target_arch "gfx1200": the reference converter's recipe (gfx12 tile order; W3
 * fragments are re-packed while loading); "gfx950": this library's recipe (loads as
 * plain copies). */
typedef struct gfxinfer_artifact gfxinfer_artifact;

/* ArtifactIdentity (artifact.h:35-40), NUL-padded as on disk. */
typedef struct gfxinfer_artifact_identity {
  char target_arch[16];
  char model_id[32];
  char weights_id[32];
  char recipe_id[64];
} gfxinfer_artifact_identity;

/* TensorDescriptor (artifact.h:42-55).  dtype: 1 u8, 2 i32, 3 f16, 4 bf16, 5 f32;
 * quantization: 0 none, 1 W2G128, 2 W3G128, 3 W4G128, 4 W8G128, 5 FP8 rows.  `name`
 * stays valid until the artifact is closed; offsets are file offsets. */
typedef struct gfxinfer_artifact_tensor {
  const char* name;
  uint16_t dtype;
  uint16_t quantization;
  uint16_t rank;
  uint16_t flags;
  uint32_t alignment;
  uint64_t dimensions[4];
  uint64_t data_offset;
  uint64_t data_bytes;
  uint64_t aux_offset;
  uint64_t aux_bytes;
  uint64_t data_crc64;
} gfxinfer_artifact_tensor;

/* ArtifactView::open (artifact.cpp:264-411): maps the file and validates magic,
 * version, byte order, section bounds, names, alignment, payload overlap and (when
 * verify_checksums is non-zero) every checksum.  GFXI_IO_ERROR, GFXI_CORRUPT_ARTIFACT
 * or GFXI_UNSUPPORTED on failure, as the reference. */
int32_t gfxinfer_artifact_open(const char* path, int32_t verify_checksums, gfxinfer_artifact** out);
void gfxinfer_artifact_close(gfxinfer_artifact* artifact);
int32_t gfxinfer_artifact_get_identity(const gfxinfer_artifact* artifact, gfxinfer_artifact_identity* out);
size_t gfxinfer_artifact_tensor_count(const gfxinfer_artifact* artifact);
int32_t gfxinfer_artifact_tensor_at(const gfxinfer_artifact* artifact, size_t index,
                                    gfxinfer_artifact_tensor* out);
/* ArtifactView::find (artifact.cpp:413-417). */
int32_t gfxinfer_artifact_find(const gfxinfer_artifact* artifact, const char* name,
                               gfxinfer_artifact_tensor* out);
/* ArtifactView::data / auxiliary (artifact.cpp:419-425): `bytes` bytes of the mapped
 * file at `offset`, or NULL outside the file. */
const void* gfxinfer_artifact_bytes(const gfxinfer_artifact* artifact, uint64_t offset, uint64_t bytes);
/* Engine::resource (engine.h:90-91, engine.cpp:229-236): the bytes of an unquantized u8
 * tensor named "resources/..." (for example "resources/tokenizer.json"), valid until the
 * artifact is closed.  GFXI_INVALID_ARGUMENT when there is no such resource. */
int32_t gfxinfer_artifact_resource(const gfxinfer_artifact* artifact, const char* name, const void** data,
                                   uint64_t* bytes);
/* crc64_ecma_update (artifact.cpp:191-213). */
uint64_t gfxinfer_crc64_ecma(uint64_t state, const void* bytes, size_t count);

/* No reference counterpart: converts codes in the reference's gfx12 tile order
 * (quantization.cpp:253-318, the "gfx1200" recipe) to the gfx950 tile layout (W2 and W3
 * fragments re-packed, W4 copied); the loader's conversion, on the host.  `bytes` is a
 * multiple of the 32-column fragment (8 B W2, 12 B W3, 16 B W4); scales need no
 * conversion. */
int32_t gfxinfer_retile_gfx12_for_gfx950(int32_t format, const uint8_t* gfx12_codes, size_t bytes,
                                         uint8_t* gfx950_codes);

/* Engine::create from an artifact (engine.cpp:62-209) for the spec's shapes: every
 * tensor of the converter's naming is required; matrices take the artifact's W3/W4
 * quantization, the rest bf16; an "mtp.draft_head.weight" + "mtp.draft_head_token_ids"
 * pair (converter.cpp:252-302) becomes the MTP draft head with its token-id map. */
int32_t gfxinfer_model_create_from_artifact(const gfxinfer_model_spec* spec, const char* path,
                                            int32_t verify_checksums, int32_t device,
                                            gfxinfer_model** out);
/* No reference counterpart (the reference writes artifacts only from safetensors): writes
 * the model's arena as a gfx950-recipe artifact (identity gfx950 / qwen3.8-27b /
 * weights_id / "gfx950-tile16x128-w3w4-bf16") through a temporary file and rename.
 * With draft_count > 0 (a multiple of 16) it also writes the converter's MTP draft head
 * (converter.cpp:252-302): LM-head rows draft_rows[0..draft_count) as
 * "mtp.draft_head.weight" and the row ids as "mtp.draft_head_token_ids". */
int32_t gfxinfer_model_write_artifact(const gfxinfer_model* model, const char* path,
                                      const char* weights_id, const uint32_t* draft_rows,
                                      size_t draft_count);

/* DecodeSessionConfig (qwen_runtime.h:23-29).  Activations are always A4G128 (the
 * reference's ActivationMode::int4).  graph_verifier_batch: 0, or 2..32 to capture the
 * MTP chain + verifier of depth graph_verifier_batch - 1 as hipGraphs.  keep_logits:
 * non-zero also writes the fp32 logits of every head projection to the "logits" buffer
 * (a test accessor; the argmax is fused into the projection either way). */
typedef struct gfxinfer_session_config {
  size_t maximum_context_tokens;
  uint32_t graph_verifier_batch;
  int32_t keep_logits;
} gfxinfer_session_config;

/* DecodeSessionSummary (qwen_runtime.h:31-37). */
typedef struct gfxinfer_session_summary {
  size_t arena_bytes;
  size_t maximum_context_tokens;
  size_t gdn_state_bytes;
  size_t kv_cache_bytes;
  size_t mtp_cache_bytes;
} gfxinfer_session_summary;

/* SpeculativeStepResult (qwen_runtime.h:39-45): token_count = accepted_drafts + 1
 * tokens, the accepted drafts then the target's correction or bonus token. */
typedef struct gfxinfer_speculative_result {
  uint32_t tokens[32];
  uint32_t token_count;
  uint32_t proposed_drafts;
  uint32_t accepted_drafts;
} gfxinfer_speculative_result;

typedef struct gfxinfer_session gfxinfer_session;

/* QwenDecodeSession::create (qwen_runtime.cpp:943-1262). */
int32_t gfxinfer_session_create(gfxinfer_model* model, const gfxinfer_session_config* config,
                                gfxinfer_session** out);
void gfxinfer_session_destroy(gfxinfer_session* session);
/* QwenDecodeSession::greedy_step (qwen_runtime.cpp:1264-1318). */
int32_t gfxinfer_session_greedy_step(gfxinfer_session* session, uint32_t input_token,
                                     uint32_t* output_token);
/* QwenDecodeSession::block_step (qwen_runtime.cpp:1320-1392): 1..32 tokens;
 * output_tokens receives one target token per input. */
int32_t gfxinfer_session_block_step(gfxinfer_session* session, const uint32_t* input_tokens,
                                    size_t count, uint32_t* output_tokens);
/* QwenDecodeSession::mtp_draft (qwen_runtime.cpp:1394-1419). */
int32_t gfxinfer_session_mtp_draft(gfxinfer_session* session, uint32_t next_token,
                                   uint32_t* output_token);
/* QwenDecodeSession::speculative_step (qwen_runtime.cpp:1421-1544): draft_count 1..31. */
int32_t gfxinfer_session_speculative_step(gfxinfer_session* session, uint32_t seed_token,
                                          size_t draft_count,
                                          gfxinfer_speculative_result* result);
/* speculative_step with an acceptance override, for benchmarks on synthetic weights
 * whose drafts never match: accepted_drafts = forced_accepted (0..draft_count) whatever
 * the comparison says; everything else (proposals, verifier, rollback or state swap,
 * MTP cache advance) runs as in speculative_step.  No reference counterpart. */
int32_t gfxinfer_session_speculative_step_forced(gfxinfer_session* session,
                                                 uint32_t seed_token, size_t draft_count,
                                                 uint32_t forced_accepted,
                                                 gfxinfer_speculative_result* result);
/* speculative_step whose verifier checks the given host drafts instead of the MTP
 * chain's (the chain still runs and advances the MTP cache).  Test hook for
 * planted-acceptance checks on synthetic weights; no reference counterpart. */
int32_t gfxinfer_session_speculative_step_planted(gfxinfer_session* session,
                                                  uint32_t seed_token, size_t draft_count,
                                                  const uint32_t* planted_drafts,
                                                  gfxinfer_speculative_result* result);
/* QwenDecodeSession::position / summary (qwen_runtime.cpp:1546-1552). */
size_t gfxinfer_session_position(const gfxinfer_session* session);
size_t gfxinfer_session_mtp_position(const gfxinfer_session* session);
int32_t gfxinfer_session_get_summary(const gfxinfer_session* session,
                                 gfxinfer_session_summary* out);
/* Copies `bytes` bytes from offset `offset` of a named session buffer into host memory
 * ("logits", "hidden", "selected", "drafts", "conv_states", "gdn_states",
 * "key_caches", "value_caches", "mtp_key_cache", "mtp_value_cache", "mtp_hidden").
 * No reference counterpart: a test accessor. */
int32_t gfxinfer_session_copy_buffer(const gfxinfer_session* session, const char* name,
                                     size_t offset, void* host, size_t bytes);
/* Byte size of a named session buffer (0 if unknown). */
size_t gfxinfer_session_buffer_bytes(const gfxinfer_session* session, const char* name);
/* Test hook, no reference counterpart: with device_trace set (NULL turns it off), every
 * eager verifier pass (block_step, greedy_step, prefill, planted rounds) copies each
 * decoder layer's stage boundaries into device_trace (at least
 * gfxinfer_session_layer_trace_bytes bytes), for stage-by-stage comparison against a CPU
 * model.  Sections, in order, each sized for 32 tokens (W = max(attention width, GDN
 * value width), I = MLP width):
 *   residual [layers + 1][32][hidden] fp16 -- rows entering layer 0, then leaving each layer;
 *   post [layers][32][hidden] fp16 -- rows after the mixer's residual add;
 *   mixer codes [layers][32 * W / 2] and scales [layers][32 * W / 128] fp16 -- the A4 input
 *     of the o / out projection, stored as [tokens][width / 2] and [tokens][width / 128];
 *   MLP codes [layers][32 * I / 2] and scales [layers][32 * I / 128] fp16 -- the A4 SwiGLU
 *     output (the down projection's input), stored the same way.
 * Captured graphs are not affected. */
size_t gfxinfer_session_layer_trace_bytes(const gfxinfer_session* session);
int32_t gfxinfer_session_set_layer_trace(gfxinfer_session* session, void* device_trace,
                                         size_t bytes);

/* Chunked prefill.  The reference prefills a prompt with one greedy_step per token and,
 * when MTP is on, an mtp_draft per token from the second on (cli/main.cpp:1055-1069);
 * this runs the target over the prompt in blocks of up to 32 tokens and, with
 * sync_mtp != 0, advances the MTP K/V cache over the same positions in batches (entry j
 * from token j + 1 and the target's hidden state at position j), leaving the target,
 * GDN, KV and MTP cache state and the positions as that serial loop leaves them.
 * *next_token = the greedy token after the last prompt token.  Requires a fresh
 * session or, with sync_mtp, an aligned one (mtp_position + 1 == position).  No
 * reference counterpart (the reference roadmap's "fast prefill", README.md:211-218). */
int32_t gfxinfer_session_prefill(gfxinfer_session* session, const uint32_t* tokens, size_t count,
                                 int32_t sync_mtp, uint32_t* next_token);

/* Online MTP depth selection ("Online MTP depth selection based on accepted tokens
 * per millisecond", docs/ROADMAP.md:51; not implemented by the reference).  The
 * policy keeps, per candidate depth {1, 2, 3, 4, 6, 8, 12, 16, 24, 31} up to
 * maximum_depth, exponential averages (weight 1/4) of tokens emitted per round and of
 * milliseconds per round; choose() returns the first untried candidate within
 * `limit`, else the one with the most tokens per millisecond, except that every 16th
 * round it re-measures one of the other candidates within `limit`, in turn.  Host
 * only, deterministic. */
typedef struct gfxinfer_depth_policy gfxinfer_depth_policy;
int32_t gfxinfer_depth_policy_create(uint32_t maximum_depth, gfxinfer_depth_policy** out);
void gfxinfer_depth_policy_destroy(gfxinfer_depth_policy* policy);
uint32_t gfxinfer_depth_policy_choose(gfxinfer_depth_policy* policy, uint32_t limit);
int32_t gfxinfer_depth_policy_record(gfxinfer_depth_policy* policy, uint32_t depth,
                                     uint32_t emitted_tokens, double milliseconds);

/* The generate loop of the reference CLI (cli/main.cpp:1023-1120) without the
 * tokenizer: prefill the prompt, then greedy steps (draft_count == 0) or speculative
 * rounds of depth min(draft_count, tokens still wanted - 1) (or the depth policy's
 * choice, adaptive_depth != 0) until maximum_tokens tokens are out or a stop token
 * was emitted.  The first output token is the prefill's greedy token. */
typedef struct gfxinfer_generate_config {
  uint32_t maximum_tokens;       /* >= 1; prompt + maximum_tokens <= the session context */
  uint32_t draft_count;          /* 0..31 */
  int32_t adaptive_depth;        /* non-zero: online depth selection up to draft_count */
  const uint32_t* stop_tokens;   /* end-of-turn ids (the reference's 248044, 248046) */
  uint32_t stop_count;
} gfxinfer_generate_config;

typedef struct gfxinfer_generate_stats {
  size_t prompt_tokens;
  size_t output_tokens;
  size_t speculative_rounds;
  size_t proposed_drafts;
  size_t accepted_drafts;
  size_t speculative_emitted;
  double prefill_ms;             /* time to first token */
  double decode_ms;              /* after the first token */
} gfxinfer_generate_stats;

/* output: capacity config->maximum_tokens; *output_count = tokens written. */
int32_t gfxinfer_session_generate(gfxinfer_session* session, const uint32_t* prompt,
                                  size_t prompt_count, const gfxinfer_generate_config* config,
                                  uint32_t* output, size_t* output_count,
                                  gfxinfer_generate_stats* stats);

/* ---- Tokenizer and chat prompt (tokenizer.h, tokenizer.cpp; cli/main.cpp) ----------
 * Byte-level BPE over a tokenizer.json document: NFC normalization, the Qwen pre-token
 * pattern, the GPT-2 byte alphabet and ranked merges, with added tokens matched in the raw
 * text.  Sizes are in bytes of UTF-8 (text) or in ids; an output buffer that is too small
 * receives a prefix and the full size is still returned, so a caller can retry. */
typedef struct gfxinfer_tokenizer gfxinfer_tokenizer;

/* QwenTokenizer::from_json (tokenizer.h:19-20, tokenizer.cpp:174-248).  Ids of the
 * vocabulary and the added tokens must cover 0 .. N-1; merges are "left right" strings or
 * [left, right] pairs.  GFXI_CORRUPT_ARTIFACT for a malformed document. */
int32_t gfxinfer_tokenizer_create(const void* json, size_t bytes, gfxinfer_tokenizer** out);
void gfxinfer_tokenizer_destroy(gfxinfer_tokenizer* tokenizer);
/* QwenTokenizer::vocabulary_size (tokenizer.h:25). */
size_t gfxinfer_tokenizer_vocabulary_size(const gfxinfer_tokenizer* tokenizer);
/* QwenTokenizer::encode (tokenizer.h:23-24, tokenizer.cpp:277-357): writes
 * min(count, capacity) ids and sets *count to the number of ids of the text. */
int32_t gfxinfer_tokenizer_encode(const gfxinfer_tokenizer* tokenizer, const char* text, size_t length,
                                  uint32_t* ids, size_t capacity, size_t* count);
/* QwenTokenizer::decode (tokenizer.h:21-22, tokenizer.cpp:250-275): writes
 * min(length, capacity) bytes (no terminator) and sets *length to the decoded size.
 * GFXI_INVALID_ARGUMENT for an id outside the vocabulary. */
int32_t gfxinfer_tokenizer_decode(const gfxinfer_tokenizer* tokenizer, const uint32_t* ids, size_t count,
                                  char* text, size_t capacity, size_t* length);
/* The generate command's chat rendering (cli/main.cpp:1037-1039): one user turn and an
 * opened assistant turn with an empty thinking block. */
int32_t gfxinfer_render_chat_prompt(const char* prompt, size_t length, char* text, size_t capacity,
                                    size_t* rendered_length);

#ifdef __cplusplus
}
#endif
#endif
