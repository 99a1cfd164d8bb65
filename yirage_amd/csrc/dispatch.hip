// Generic fused-operator launcher with the argument shape of the reference's
// execute_mugraph(inputs, outputs, buffer, stream, profiler)
// (python/yirage/kernel.py:22-72,411-421).
#include <string.h>

#include "yr_common.h"

using namespace yr;

extern "C" int yr_hip_run_fused(int op_kind, int n_in, const void* const* in, int n_out, void* const* out,
                                int n_params, const int64_t* p, void* workspace, size_t workspace_bytes,
                                void* stream) {
  const char* nm = "yr_hip_run_fused";
  if ((n_in && !in) || (n_out && !out) || (n_params && !p)) return fail(YR_E_INVALID, "%s: null array", nm);
  switch (op_kind) {
    case YR_OP_RMSNORM_LINEAR: {
      if (n_in != 3 || n_out != 1 || n_params != 6) return fail(YR_E_INVALID, "%s: rmsnorm_linear arity", nm);
      float eps;
      int32_t bits = (int32_t)p[5];
      memcpy(&eps, &bits, 4);
      return yr_hip_rmsnorm_linear(in[0], in[1], in[2], out[0], (int)p[0], (int)p[1], (int)p[2], (int)p[3],
                                   (int)p[4], eps, workspace, workspace_bytes, stream);
    }
    case YR_OP_GATED_MLP:
      if (n_in != 3 || n_out != 1 || n_params != 5) return fail(YR_E_INVALID, "%s: gated_mlp arity", nm);
      return yr_hip_gated_mlp(in[0], in[1], in[2], out[0], (int)p[0], (int)p[1], (int)p[2], (int)p[3], (int)p[4],
                              workspace, workspace_bytes, stream);
    case YR_OP_GQA_PREFILL:
      if (n_in != 3 || n_out != 1 || n_params != 7) return fail(YR_E_INVALID, "%s: gqa_prefill arity", nm);
      return yr_hip_gqa_prefill(in[0], in[1], in[2], out[0], (int)p[0], (int)p[1], (int)p[2], (int)p[3],
                                (int)p[4], (int)p[5], (int)p[6], stream);
    case YR_OP_LINEAR:
      if (n_in != 3 || n_out != 1 || n_params != 5) return fail(YR_E_INVALID, "%s: linear arity", nm);
      return yr_hip_linear(in[0], in[1], in[2], out[0], (int)p[0], (int)p[1], (int)p[2], (int)p[3], (int)p[4],
                           workspace, workspace_bytes, stream);
    default:
      return fail(YR_E_INVALID, "%s: unknown op kind %d", nm, op_kind);
  }
}
