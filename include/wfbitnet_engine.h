/*
 * wfbitnet_engine.h - native greedy/top-p BitNet engine on the MI355X kernels of libwfbitnet.
 *
 * The C ABI of the reference's native engine, same names, structs and error behaviour, so the
 * Rust gateway's FFI (SGB/sgl-model-gateway/src/inference/bitnet_ffi.rs:55-100) binds it unchanged
 * after linking libwfbitnet.so in place of sgl_kernel_inference.  Replaces
 * SGB/sgl-kernel/csrc/inference/bitnet_engine.h:14-161 (implementation bitnet_engine.cpp).
 *
 * Model: an SGLBITNT file (the format of SGB/sgl-kernel/csrc/inference/sglkernel_loader.h:1-161,
 * written by packages/inference/scripts/convert_to_sglkernel.py); packed linears are I2_S uint8
 * [out, k_pad/4] with their per-tensor scale, K padded to a multiple of 128; embedding, norms and a
 * dense LM head in float32 / float16 / bfloat16 (held as bfloat16 on the GPU); a uint8 lm_head.weight
 * is a ternary head, none a head tied to the embedding.  The layer is the stage-1 BitNet form (the
 * intent the reference engine states, with the rotary embedding its attention_forward omits):
 * RMSNorm -> q|k|v BitLinears -> HF rotary embedding -> causal GQA attention over a bf16 KV cache ->
 * SubLN -> o BitLinear + residual -> RMSNorm -> gate|up BitLinears -> act(gate) * up (hidden_act
 * "silu" or "relu2") -> SubLN -> down BitLinear + residual; final RMSNorm and the LM head.  Config
 * keys read from the file's JSON: vocab_size, hidden_size, intermediate_size, num_hidden_layers,
 * num_attention_heads, num_key_value_heads (default: heads), head_dim (default hidden / heads; 64 or
 * 128), rope_theta (10000), rms_norm_eps (1e-5), subln_eps (1e-6), hidden_act ("silu"),
 * max_position_embeddings (4096), eos_token_id (none when absent).
 *
 * Execution: one engine owns one HIP stream on the device current at bitnet_engine_create and
 * keeps every weight, the KV cache and its work buffers in that device's memory.  A prompt runs as
 * one batched pass (the prefill GEMMs and the matrix-core prefill attention); every later token is
 * one replay of a captured HIP graph.  Every call returns only when its work on the GPU is done.
 * One engine must not be used from two threads at once.
 *
 * SGB = packages/inference/extern/sglang-bitnet (paths as in wfbitnet.h).
 */
#ifndef WFBITNET_ENGINE_H
#define WFBITNET_ENGINE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Opaque engine handle (bitnet_engine.h:19). */
typedef struct BitNetEngine BitNetEngine;

/* Engine configuration (bitnet_engine.h:22-26).  max_seq_len > 0 overrides the file's
 * max_position_embeddings (KV cache positions); num_threads and kv_cache_size are accepted and
 * ignored (the engine runs on the GPU; the cache is sized by max_seq_len). */
typedef struct {
    int32_t max_seq_len;
    int32_t num_threads;
    int32_t kv_cache_size;
} BitNetConfig;

/* Sampling parameters (bitnet_engine.h:29-35).  temperature <= 0: greedy (first maximal logit);
 * else top-p sampling of softmax(logits / temperature) (top_p <= 0 means 1) with the engine's
 * std::mt19937 seeded 42 at creation, as the reference's sample_top_p (bitnet_engine.cpp:221-253), except
 * where float rounding leaves the running sum of all probabilities below top_p: the reference then
 * keeps only the most probable token, here every token is kept.  top_k and repetition_penalty are
 * accepted and, as in the reference engine, not applied. */
typedef struct {
    float temperature;
    float top_p;
    int32_t top_k;
    float repetition_penalty;
    int32_t max_tokens;
} SamplingParams;

/* Generation result (bitnet_engine.h:38-43): output_ids malloc'd by the library, freed with
 * bitnet_free_result; logits is always NULL (logits_size 0), as in the reference. */
typedef struct {
    int32_t* output_ids;
    int32_t num_tokens;
    float* logits;
    int32_t logits_size;
} GenerationResult;

/* Load an SGLBITNT model onto the current HIP device (bitnet_engine.h:56; bitnet_engine.cpp:681-732).
 * NULL on error, with the reason in bitnet_get_error(): unreadable file, bad magic or version, a
 * missing tensor, a shape that does not match the config, or a configuration the kernels do not
 * take (head_dim other than 64/128, more than 8 query heads per kv head, hidden_act other than
 * silu/relu2, a row length not a multiple of 8, device memory exhausted). */
BitNetEngine* bitnet_engine_create(const char* model_path, const BitNetConfig* config);

/* Free the engine and its device memory (bitnet_engine.h:61; bitnet_engine.cpp:734-736; NULL is ignored). */
void bitnet_engine_destroy(BitNetEngine* engine);

/* Message of the last failed engine call on this thread (bitnet_engine.h:67; thread-local as in
 * bitnet_engine.cpp:86, 738-740). */
const char* bitnet_get_error(void);

/* Reset the cache, run the prompt, then produce up to params->max_tokens tokens, stopping after the
 * first eos_token_id (bitnet_engine.h:83-89; bitnet_engine.cpp:742-823).  Every produced token is
 * also run through the model, so afterwards the engine stands where the reference's would: the next
 * bitnet_decode_step picks from the logits of the last token run.  0 on success, -1 on error:
 * engine or params NULL, num_input_tokens < 1, a token id outside [0, vocab), or
 * num_input_tokens + max_tokens above max_seq_len. */
int bitnet_generate(BitNetEngine* engine, const int32_t* input_ids, int32_t num_input_tokens,
                    const SamplingParams* params, GenerationResult* result);

/* Reset the cache and run the prompt (positions 0 .. num_tokens-1) in one batched pass
 * (bitnet_engine.h:99-103; bitnet_engine.cpp:825-849).  0 / -1 (num_tokens < 1, ids out of range,
 * num_tokens > max_seq_len). */
int bitnet_prefill(BitNetEngine* engine, const int32_t* input_ids, int32_t num_tokens);

/* Pick the next token from the logits of the last token run (greedy or sampled per params), store it
 * in *output_id, and run it through the model at `position` (bitnet_engine.h:114-119;
 * bitnet_engine.cpp:851-893).  0 / -1 (no prompt run since creation or the last reset, position
 * outside [0, max_seq_len)).  A failure of the GPU work of a step or of a generation leaves no pending
 * state: the next decode step needs a new prompt. */
int bitnet_decode_step(BitNetEngine* engine, int32_t position, const SamplingParams* params, int32_t* output_id);

/* Forget the sequence (bitnet_engine.h:124; bitnet_engine.cpp:895-900). */
void bitnet_reset_cache(BitNetEngine* engine);

/* Model information (bitnet_engine.h:133-148; bitnet_engine.cpp:902-916; 0 for a NULL engine). */
int32_t bitnet_vocab_size(BitNetEngine* engine);
int32_t bitnet_hidden_size(BitNetEngine* engine);
int32_t bitnet_num_layers(BitNetEngine* engine);
int32_t bitnet_max_seq_len(BitNetEngine* engine);
/* Number of kv heads (exported by bitnet_engine.cpp:918-920 without a declaration in its header). */
int bitnet_get_num_kv_heads(BitNetEngine* engine);

/* Free output_ids / logits of a result and clear them (bitnet_engine.h:157; bitnet_engine.cpp:922-929). */
void bitnet_free_result(GenerationResult* result);

/* The engine's top-p sampler on host logits, for tests: `draws` picks from the same logits [n] with a
 * fresh std::mt19937(seed), each exactly as bitnet_decode_step samples (softmax of logits / temperature
 * in float32, probabilities sorted in descending order, the shortest prefix whose running sum reaches
 * top_p or else all of them, a uniform float in [0, that sum) located in the prefix).  No counterpart in the reference's
 * ABI.  0, or -1 for n < 1, temperature <= 0, draws < 0 or NULL pointers. */
int wfb_engine_sample_top_p(const float* logits, int64_t n, float temperature, float top_p, uint32_t seed,
                            int32_t draws, int32_t* out);

/* Test hook, no counterpart in the reference's ABI: after `n` more successful allocations the engine's
 * allocator (device buffers and the prompt's pinned id buffer) reports one failure, then allocates normally
 * again; n < 0 (the default) never fails.  Process-wide.  Lets tests reach the out-of-memory paths, e.g. a
 * prompt longer than any before it whose buffer growth fails: that call returns -1 and leaves no buffers,
 * and the next prompt allocates again.  Returns 0. */
int wfb_engine_fail_alloc_after(int64_t n);

#ifdef __cplusplus
}
#endif

#endif /* WFBITNET_ENGINE_H */
