// Internal (C++) launchers of the attention kernels, shared by the C-ABI
// entry points and the kernel-graph operators: the same kernels with an
// explicit softmax scale and, for prefill, explicit strides.
#pragma once
#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

namespace yr {

// Paged GQA decode (q[batch][hq][d], caches [pages][page_size][hkv][d]);
// `workspace` holds workspace_bytes >= yr_hip_gqa_decode_workspace(...).
int gqa_decode_launch(const char* nm, const void* q, const void* k_cache, const void* v_cache,
                      const int32_t* kv_indptr, const int32_t* kv_indices, const int32_t* kv_len, void* out,
                      int batch, int hq, int hkv, int d, int page_size, int max_kv_len, int dtype, void* workspace,
                      size_t workspace_bytes, hipStream_t st, float scale);

// The shape / dtype checks of gqa_decode_launch (all but the workspace).
int gqa_decode_check(const char* nm, const void* q, const void* k_cache, const void* v_cache,
                     const int32_t* kv_indptr, const int32_t* kv_indices, const int32_t* kv_len, const void* out,
                     int batch, int hq, int hkv, int d, int page_size, int max_kv_len, int dtype);

// Flash-attention prefill over batch x heads with sq query rows and sk kv
// rows per batch entry; strides in elements.
int prefill_launch(const char* nm, const void* q, const void* k, const void* v, void* out, int batch, int sq, int sk,
                   int hq, int hkv, int d, int causal, int dtype, long long q_bs, int q_ld, long long kv_bs, int kv_ld,
                   long long o_bs, int o_ld, float scale, hipStream_t st);

}  // namespace yr
