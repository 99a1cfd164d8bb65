// Generic fused-operator launcher with the argument shape of the reference's
// execute_mugraph(inputs, outputs, buffer, stream, profiler)
// (python/yirage/kernel.py:22-72,411-421): the kernel-graph front end turns
// a graph into a list of (op kind, inputs, outputs, integer params) steps and
// runs each one through yr_hip_run_fused on a shared workspace.
#include <string.h>

#include "yr_common.h"

using namespace yr;

namespace {

float f32_of(int64_t bits) {
  float f;
  const int32_t b = (int32_t)bits;
  memcpy(&f, &b, 4);
  return f;
}

struct Arity {
  int n_in, n_out, n_params;  // n_params < 0: at least -n_params
};

bool arity_of(int kind, Arity* a) {
  switch (kind) {
    case YR_OP_RMSNORM_LINEAR: *a = {3, 1, 6}; return true;
    case YR_OP_GATED_MLP: *a = {3, 1, 5}; return true;
    case YR_OP_GQA_PREFILL: *a = {3, 1, 7}; return true;
    case YR_OP_LINEAR: *a = {3, 1, 5}; return true;
    case YR_OP_GQA_DECODE: *a = {6, 1, 7}; return true;
    case YR_OP_ATTENTION: *a = {3, 1, 18}; return true;
    case YR_OP_MATMUL: *a = {2, 1, 5}; return true;
    case YR_OP_UNARY: *a = {1, 1, 5}; return true;
    case YR_OP_BINARY: *a = {2, 1, -3}; return true;
    case YR_OP_REDUCTION: *a = {1, 1, 4}; return true;
    case YR_OP_RMSNORM: *a = {1, 1, 4}; return true;
    case YR_OP_PACK: *a = {1, 1, 11}; return true;
    case YR_OP_COPY_ND: *a = {1, 1, -27}; return true;  // 27, or 28 with a source offset
    case YR_OP_REDUCTION_MAX: *a = {1, 1, 4}; return true;
    case YR_OP_EWISE: *a = {-1, 1, -4}; return true;  // 1..8 inputs
    case YR_OP_TB_PROGRAM: *a = {-1, -1, -16}; return true;  // 1..8 inputs, 1..4 outputs
    default: return false;
  }
}

}  // namespace

extern "C" {

size_t yr_hip_fused_workspace(int op_kind, int n_params, const int64_t* p) {
  Arity ar;
  if (!arity_of(op_kind, &ar) || (n_params && !p)) return 0;
  if (ar.n_params >= 0 ? n_params != ar.n_params : n_params < -ar.n_params) return 0;
  switch (op_kind) {
    case YR_OP_RMSNORM_LINEAR:
      return yr_hip_rmsnorm_linear_workspace((int)p[0], (int)p[1], (int)p[2], (int)p[3], (int)p[4]);
    case YR_OP_GATED_MLP:
      return yr_hip_gated_mlp_workspace((int)p[0], (int)p[1], (int)p[2], (int)p[3], (int)p[4]);
    case YR_OP_LINEAR:
      return yr_hip_linear_workspace((int)p[0], (int)p[1], (int)p[2], (int)p[3], (int)p[4]);
    case YR_OP_GQA_DECODE:
      return yr_hip_gqa_decode_workspace((int)p[0], (int)p[1], (int)p[2], (int)p[3], (int)p[5], (int)p[4]);
    case YR_OP_ATTENTION:
      return yr_hip_graph_attention_workspace((int)p[0], (int)p[1], (int)p[2], (int)p[3], p + 6);
    default:
      return 0;
  }
}

int yr_hip_run_fused(int op_kind, int n_in, const void* const* in, int n_out, void* const* out, int n_params,
                     const int64_t* p, void* workspace, size_t workspace_bytes, void* stream) {
  const char* nm = "yr_hip_run_fused";
  if ((n_in && !in) || (n_out && !out) || (n_params && !p)) return fail(YR_E_INVALID, "%s: null array", nm);
  Arity ar;
  if (!arity_of(op_kind, &ar)) return fail(YR_E_INVALID, "%s: unknown op kind %d", nm, op_kind);
  if ((ar.n_in >= 0 ? n_in != ar.n_in : n_in < 1) || (ar.n_out >= 0 ? n_out != ar.n_out : n_out < 1) ||
      (ar.n_params >= 0 ? n_params != ar.n_params : n_params < -ar.n_params))
    return fail(YR_E_INVALID, "%s: op kind %d takes %s%d inputs, %d outputs and %s%d params (got %d, %d, %d)", nm,
                op_kind, ar.n_in < 0 ? ">= " : "", ar.n_in < 0 ? 1 : ar.n_in, ar.n_out, ar.n_params < 0 ? ">= " : "", ar.n_params < 0 ? -ar.n_params : ar.n_params,
                n_in, n_out, n_params);
  switch (op_kind) {
    case YR_OP_RMSNORM_LINEAR:
      return yr_hip_rmsnorm_linear(in[0], in[1], in[2], out[0], (int)p[0], (int)p[1], (int)p[2], (int)p[3],
                                   (int)p[4], f32_of(p[5]), workspace, workspace_bytes, stream);
    case YR_OP_GATED_MLP:
      return yr_hip_gated_mlp(in[0], in[1], in[2], out[0], (int)p[0], (int)p[1], (int)p[2], (int)p[3], (int)p[4],
                              workspace, workspace_bytes, stream);
    case YR_OP_GQA_PREFILL:
      return yr_hip_gqa_prefill(in[0], in[1], in[2], out[0], (int)p[0], (int)p[1], (int)p[2], (int)p[3],
                                (int)p[4], (int)p[5], (int)p[6], stream);
    case YR_OP_LINEAR:
      return yr_hip_linear(in[0], in[1], in[2], out[0], (int)p[0], (int)p[1], (int)p[2], (int)p[3], (int)p[4],
                           workspace, workspace_bytes, stream);
    case YR_OP_GQA_DECODE:
      return yr_hip_gqa_decode_paged(in[0], in[1], in[2], (const int32_t*)in[3], (const int32_t*)in[4],
                                     (const int32_t*)in[5], out[0], (int)p[0], (int)p[1], (int)p[2], (int)p[3],
                                     (int)p[4], (int)p[5], (int)p[6], workspace, workspace_bytes, stream);
    case YR_OP_ATTENTION:
      return yr_hip_graph_attention(in[0], in[1], in[2], out[0], (int)p[0], (int)p[1], (int)p[2], (int)p[3], p + 6,
                                    f32_of(p[5]), (int)p[4], workspace, workspace_bytes, stream);
    case YR_OP_MATMUL:
      return yr_hip_graph_matmul(in[0], in[1], out[0], (int)p[0], (int)p[1], (int)p[2], (int)p[3], (int)p[4], stream);
    case YR_OP_UNARY:
      return yr_hip_graph_unary(in[0], out[0], p[0], (int)p[1], f32_of(p[3]), f32_of(p[4]), (int)p[2], stream);
    case YR_OP_BINARY: {
      const int nd = (int)p[0];
      if (nd < 1 || n_params != 3 + 2 * nd) return fail(YR_E_INVALID, "%s: binary takes 3 + 2 ndim params", nm);
      return yr_hip_graph_binary(in[0], in[1], out[0], nd, p + 3, p + 3 + nd, (int)p[1], (int)p[2], stream);
    }
    case YR_OP_REDUCTION:
      return yr_hip_graph_reduction(in[0], out[0], p[0], (int)p[1], p[2], (int)p[3], stream);
    case YR_OP_RMSNORM:
      return yr_hip_graph_rmsnorm(in[0], out[0], (int)p[0], (int)p[1], f32_of(p[3]), (int)p[2], stream);
    case YR_OP_PACK:
      return yr_hip_graph_pack(in[0], out[0], (int)p[0], (int)p[1], (int)p[2], (int)p[3], p + 5, (int)p[4], stream);
    case YR_OP_COPY_ND:  // p[26]: element offset of the destination; p[27] (optional): of the source
      if (n_params > 28) return fail(YR_E_INVALID, "%s: copy_nd takes 27 or 28 params", nm);
      return yr_hip_graph_copy_nd(in[0] ? (const uint16_t*)in[0] + (n_params > 27 ? p[27] : 0) : nullptr,
                                  out[0] ? (uint16_t*)out[0] + p[26] : nullptr, (int)p[0], p + 2, p + 10, p + 18,
                                  (int)p[1], stream);
    case YR_OP_REDUCTION_MAX:
      return yr_hip_graph_reduction_max(in[0], out[0], p[0], (int)p[1], p[2], (int)p[3], stream);
    case YR_OP_TB_PROGRAM: {
      int32_t w[800];
      const int nw = n_params - 4;
      if (nw > 800) return fail(YR_E_INVALID, "%s: tile program of %d words (<= 800)", nm, nw);
      for (int i = 0; i < nw; i++) w[i] = (int32_t)p[4 + i];
      return yr_hip_tb_program(w, nw, in, n_in, out, n_out, (int)p[0], (int)p[1], (int)p[2], (int)p[3], stream);
    }
    case YR_OP_EWISE: {
      // {ndim, n_in, n_prog, dtype, out_dims[ndim], in_dims[n_in][ndim], prog[n_prog][5], imm_bits[n_prog][2]}
      const int nd = (int)p[0], ni = (int)p[1], np = (int)p[2];
      if (nd < 1 || nd > 6 || ni < 1 || ni > 8 || np < 1 || np > 32 || ni != n_in ||
          n_params != 4 + nd + ni * nd + 7 * np)
        return fail(YR_E_INVALID, "%s: fused elementwise params do not match their counts", nm);
      int32_t prog[32 * 5];
      float imm[32 * 2];
      const int64_t* pp = p + 4 + nd + ni * nd;
      for (int i = 0; i < 5 * np; i++) prog[i] = (int32_t)pp[i];
      for (int i = 0; i < 2 * np; i++) imm[i] = f32_of(pp[5 * np + i]);
      return yr_hip_graph_ewise(in, ni, out[0], nd, p + 4, p + 4 + nd, np, prog, imm, (int)p[3], stream);
    }
    default:
      return fail(YR_E_INVALID, "%s: unknown op kind %d", nm, op_kind);
  }
}

}  // extern "C"
