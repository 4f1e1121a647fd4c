// it_prefill.hip -- chunked-prefill attention over the paged cache (MFMA).
#include <hip/hip_runtime.h>

#include "it_internal.hpp"

using namespace itkv;

extern "C" int32_t it_paged_prefill(const it_kv_cache* c, const void* q, int32_t q_dtype, int32_t n_heads,
                                    const int32_t* cu_q, int32_t max_q_len, const int32_t* block_tables,
                                    int32_t max_blocks, const int32_t* ctx_lens, int32_t n_seqs, float scale,
                                    int32_t causal, void* out, int32_t out_dtype, void* stream) {
  return fail(IT_NOT_IMPLEMENTED, "it_paged_prefill: not built yet");
}
