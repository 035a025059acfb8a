/* libtinyinfer_llm.so — GPT-2 native runtime ABI, MI355X implementation.
 * Replaces reference llm/include/tinyinfer_llm.h:12-60 (definitions at
 * reference llm/src/runtime.cu:176-211).  Struct layouts, status codes and
 * semantics are kept so that llm/runtime.py (ctypes table at reference
 * llm/runtime.py:61-71) and the epoll server (reference
 * server/include/model.hpp:19-68) bind it unchanged.
 *
 * Synchronous HOST API: every token / logit / output pointer is a host pointer.
 * One context owns its HIP stream, weights, KV slots and scratch.  Calls on one
 * context must be serialized; contexts share nothing.  Validation failures
 * enqueue nothing and leave slot lengths unchanged; device or internal failures
 * poison the context until it is destroyed. */
#ifndef TINYINFER_LLM_H
#define TINYINFER_LLM_H
#include <stdint.h>
#ifdef __cplusplus
extern "C" {
#endif
typedef struct ti_llm_model ti_llm_model;
enum ti_llm_status { TI_LLM_OK = 0, TI_LLM_INVALID = 1, TI_LLM_IO = 2, TI_LLM_CUDA = 3,
                     TI_LLM_INTERNAL = 4 };
/* 28 bytes (reference llm/tests/test_contracts.py:141). */
typedef struct ti_llm_options {
  uint32_t struct_size; /* sizeof(ti_llm_options) */
  int32_t device, max_batch, cache_slots, capacity;
  int32_t gemm_config, attention_config;
} ti_llm_options;
/* 96 bytes, field order of reference llm/include/tinyinfer_llm.h:20-23. */
typedef struct ti_llm_trace {
  uint64_t forward_calls, embedding, gemm_fp16, gemm_int8, layernorm;
  uint64_t gelu, attention, residual, kv_scatter_gather, lm_head, argmax, nll;
} ti_llm_trace;
int ti_llm_abi_version(void); /* 1 */
const char* ti_llm_last_error(void);
int ti_llm_create(const char* manifest_path, const ti_llm_options*, ti_llm_model** out);
int ti_llm_destroy(ti_llm_model*);
int ti_llm_reset(ti_llm_model*, int32_t slot);
int ti_llm_lengths(ti_llm_model*, int32_t* out, int32_t count);
int ti_llm_get_trace(ti_llm_model*, ti_llm_trace* out);
/* Append tokens[B,token_stride] (lengths[B] > 0) to distinct slots at absolute
 * positions starting at each slot's length.  last_logits (fp32 [B,vocab]) and
 * next_tokens (greedy argmax, lowest id on ties) are optional. */
int ti_llm_forward_batch(ti_llm_model*, const int32_t* slots, const int32_t* tokens,
                         const int32_t* lengths, int32_t batch, int32_t token_stride,
                         float* last_logits, int32_t* next_tokens);
/* Greedy decode from empty distinct slots; every request generates exactly
 * max_new_tokens[b] tokens; the last generated token is not appended.  A
 * prompt id outside the vocabulary returns TI_LLM_INVALID before any work.  A
 * generated id outside it (INT_MAX, the argmax of a row whose logits are all
 * NaN, as in reference llm/src/runtime.cu:59-66) ends the call with
 * TI_LLM_INVALID after writing the tokens up to and including that step, with
 * the slot lengths advanced by the forwards that ran; the context stays usable
 * (the reference's next forward rejects the id, llm/src/runtime.cu:160). */
int ti_llm_greedy_batch(ti_llm_model*, const int32_t* slots, const int32_t* prompts,
                        const int32_t* prompt_lengths, const int32_t* max_new_tokens,
                        int32_t batch, int32_t prompt_stride, int32_t* output,
                        int32_t output_stride, int32_t* output_lengths, double* ttft_ms,
                        double* total_ms);
/* Teacher-forced NLL of one window on an internal slot (public slots untouched). */
int ti_llm_score_window(ti_llm_model*, const int32_t* tokens, const uint8_t* mask,
                        int32_t length, double* sum_nll, uint64_t* target_count,
                        double* loss_by_position);
#ifdef __cplusplus
}
#endif
#endif
