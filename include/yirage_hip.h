/*
 * yirage_hip.h -- C ABI of the MI355X-native `hip` backend for YiRage.
 *
 * Plain pointers and sizes only: no STL, no torch, no HIP types in the
 * signatures (streams travel as `void*` holding a hipStream_t; NULL is the
 * null stream).  Every entry point returns YR_OK (0) or a negative YR_E* code;
 * yr_hip_last_error() returns the message of the last failure on the calling
 * thread.  Device pointers must be 16-byte aligned.  All compute calls are
 * stream-ordered and never synchronize the device.
 *
 * Each declaration names the reference interface it replaces
 * (paths relative to the YiRage source tree).
 */
#ifndef YIRAGE_HIP_H_
#define YIRAGE_HIP_H_

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ------------------------------------------------------------------ codes */
#define YR_OK 0
#define YR_E_INVALID (-1)     /* bad argument / unsupported shape */
#define YR_E_HIP (-2)         /* HIP runtime error */
#define YR_E_WORKSPACE (-3)   /* workspace too small */
#define YR_E_NODEVICE (-4)    /* no usable gfx950 device */
#define YR_E_GRAPH (-5)       /* malformed task graph */
#define YR_E_TIMEOUT (-6)     /* persistent kernel watchdog fired */

/* dtypes: values mirror yirage::type::DataType (include/yirage/type.h:84-120) */
#define YR_DTYPE_F16 940
#define YR_DTYPE_BF16 941
#define YR_DTYPE_F32 950
#define YR_DTYPE_I32 955
#define YR_DTYPE_I64 965

/* weight layouts of a linear / matmul operand */
#define YR_W_NK 0 /* W[N][K]: torch Linear.weight, MPK linear task (tasks/ampere/linear.cuh:38-49) */
#define YR_W_KN 1 /* W[K][N]: kernel-graph matmul X @ W (src/kernel/matmul.cc:73-96) */

/* ------------------------------------------------------------------ status */
/* Message of the last failure on this thread ("" if none). */
const char* yr_hip_last_error(void);

/* Library version string. */
const char* yr_hip_version(void);

typedef struct {
  int device_id;
  int num_compute_units;      /* CUs */
  int compute_capability;     /* 950 for gfx950 */
  int wavefront_size;         /* 64 */
  size_t total_memory;        /* bytes of HBM */
  size_t max_shared_memory;   /* LDS bytes per workgroup */
  int clock_khz;
  char arch_name[64];         /* e.g. "gfx950:sramecc+:xnack-" */
} yr_device_info;

/* Replaces BackendInterface::get_info / get_num_compute_units /
 * get_compute_capability / get_max_shared_memory
 * (include/yirage/backend/backend_interface.h:74,171,184,190). */
int yr_hip_device_info(int device_id, yr_device_info* out);

/* ------------------------------------------------------- synthetic data */
/* Deterministic ~N(0, std) fill (Irwin-Hall of four 16-bit uniforms from a
 * splitmix64 counter hash; bit-identical to the CPU generator).  Used to
 * build random-init model weights on the device.  No reference counterpart
 * (the reference draws torch.randn on the host). */
int yr_hip_synth_fill(void* dst, size_t n, int dtype, uint64_t seed, uint64_t offset, float stddev,
                      void* stream);

/* ------------------------------------------------------- fused operators */
/* Workspace bytes a fused operator needs for the given shape (0 if none).
 * The workspace must be zero-filled once when it is allocated; the kernels
 * leave it zeroed again when they finish.  Replaces the buffer sizing of
 * the generated program (python/yirage/kernel.py:393-402,411-421). */
size_t yr_hip_rmsnorm_linear_workspace(int batch, int k, int n, int dtype, int w_layout);
size_t yr_hip_gated_mlp_workspace(int batch, int k, int n, int dtype, int w_layout);

/* out[b][n] = sum_k (x[b][k] * rsqrt(mean_k x[b]^2 + eps) * gamma[k]) * W(k, n)
 * fp32 accumulate, out in `dtype`.  gamma may be NULL (no affine).
 * Replaces the fused customized op found by superoptimize for
 * matmul(rms_norm(X), W) (demo/reference_mugraphs/rms_norm.py:16-25,
 * src/transpiler/transpile.cc:681-693) and the MPK task rmsnorm_linear
 * (src/kernel/task_register.cc:126-168). */
int yr_hip_rmsnorm_linear(const void* x, const void* gamma, const void* w, void* out, int batch, int k,
                          int n, int dtype, int w_layout, float eps, void* workspace,
                          size_t workspace_bytes, void* stream);

/* out[b][n] = silu(sum_k x[b][k] W1(k,n)) * (sum_k x[b][k] W3(k,n)), fp32 math.
 * Replaces the fused gated-MLP customized op
 * (demo/reference_mugraphs/gated_mlp.py:75-86). */
int yr_hip_gated_mlp(const void* x, const void* w1, const void* w3, void* out, int batch, int k, int n,
                     int dtype, int w_layout, void* workspace, size_t workspace_bytes, void* stream);

/* out[b][n] = sum_k x[b][k] W(k,n) (+ residual[b][n]), fp32 accumulate.
 * Replaces the MPK linear / linear_with_residual tasks
 * (tasks/ampere/linear_cutlass.cuh:34-475, task_register.cc:497-553). */
int yr_hip_linear(const void* x, const void* w, const void* residual, void* out, int batch, int k,
                  int n, int dtype, int w_layout, void* workspace, size_t workspace_bytes,
                  void* stream);
size_t yr_hip_linear_workspace(int batch, int k, int n, int dtype, int w_layout);

/* Paged GQA decode, one query token per sequence.
 * q[batch][hq][d]; k_cache/v_cache[num_pages][page_size][hkv][d];
 * sequence b owns pages kv_indices[kv_indptr[b] .. kv_indptr[b+1]) and has
 * kv_len[b] tokens; out[batch][hq][d] = softmax(q k^T / sqrt(d)) v with kv
 * head h / (hq / hkv).  Replaces the attention part of the MPK paged
 * attention task (tasks/ampere/multitoken_paged_attention_4_16.cuh:40-656)
 * and the superoptimize GQA customized ops
 * (demo/reference_mugraphs/group_query_attention.py:10-34). */
size_t yr_hip_gqa_decode_workspace(int batch, int hq, int hkv, int d, int max_kv_len, int page_size);
int yr_hip_gqa_decode_paged(const void* q, const void* k_cache, const void* v_cache,
                            const int32_t* kv_indptr, const int32_t* kv_indices,
                            const int32_t* kv_len, void* out, int batch, int hq, int hkv, int d,
                            int page_size, int max_kv_len, int dtype, void* workspace,
                            size_t workspace_bytes, void* stream);

/* yr_hip_gqa_decode_paged without a workspace argument and without any
 * allocation: its tickets and split records live in a fixed device array of
 * yr_hip_gqa_decode_noalloc_max_bytes() bytes per GPU (held until the
 * process ends).  Shapes needing more scratch are rejected with
 * YR_E_WORKSPACE.  Every call on one GPU shares that array, so calls that
 * overlap on one GPU (different streams, threads) race; serialize them.
 * No counterpart in the reference: it is for callers that cannot allocate
 * (code under HIP graph capture, tight serving loops, harnesses that forbid
 * hipMalloc).  Results are bit-identical to yr_hip_gqa_decode_paged. */
size_t yr_hip_gqa_decode_noalloc_max_bytes(void);
int yr_hip_gqa_decode_paged_noalloc(const void* q, const void* k_cache, const void* v_cache,
                                    const int32_t* kv_indptr, const int32_t* kv_indices,
                                    const int32_t* kv_len, void* out, int batch, int hq, int hkv, int d,
                                    int page_size, int max_kv_len, int dtype, void* stream);

/* Causal (or full) GQA prefill attention, q[batch][seq][hq][d],
 * k/v[batch][seq][hkv][d], out like q; fp32 softmax statistics, MFMA
 * contractions.  Replaces the prefill path of the MPK attention task
 * (multitoken_paged_attention_4_16.cuh:227-655 with seq_len == num_tokens). */
int yr_hip_gqa_prefill(const void* q, const void* k, const void* v, void* out, int batch, int seq,
                       int hq, int hkv, int d, int causal, int dtype, void* stream);

/* Row-wise argmax over the first n_valid of n columns of a 16-bit matrix,
 * lowest index on ties; out is int64[rows].  Replaces argmax_partial /
 * argmax_reduce (tasks/ampere/argmax.cuh:71-155). */
int yr_hip_argmax(const void* x, int64_t* out, int rows, int n, int n_valid, int dtype, void* stream);

/* ------------------------------------------------------- kernel-graph operators */
/* The operators of the reference's kernel graph (python/yirage/kernel.py:
 * 248-321; shape rules src/kernel/{matmul,element_unary,element_binary,
 * reduction,rms_norm}.cc) for the parts of a graph that no fused pattern
 * covers.  16-bit storage (f16 / bf16), fp32 math, one rounding per op, dense
 * row-major tensors unless a stride list says otherwise. */

/* Kernel-graph attention O[g] = softmax(scale * Q[g] K[g]) V[g] with
 * Q [G][M][d], K [G][d][L] (the graph's matmul operand: rows are head dims),
 * V [G][L][d] and O [G][M][d], each given by three element strides in
 * strides12 = {q0,q1,q2, k0,k1,k2, v0,v1,v2, o0,o1,o2}; d <= 128, d % 8 == 0.
 * The pattern matmul(div(exp(matmul(Q,K)), reduction(exp(.),2)), V) of
 * benchmark/group_query_attention.py:37-46 and
 * demo/reference_mugraphs/group_query_attention.py:10-34 (the reference's
 * graph has no scale: scale = 1). */
size_t yr_hip_graph_attention_workspace(int G, int M, int L, int d, const int64_t* strides12);
int yr_hip_graph_attention(const void* q, const void* k, const void* v, void* out, int G, int M, int L, int d,
                           const int64_t* strides12, float scale, int dtype, void* workspace,
                           size_t workspace_bytes, void* stream);
/* dst[i][r][c] = c < cols ? src[i s0 + r s1 + c s2] : 0 for c < dst_cols, at
 * dst + i d0 + r d1 + c d2; strides6 = {s0,s1,s2,d0,d1,d2}.  Makes strided
 * (e.g. column-major, kernel.py:196-210) graph inputs dense. */
int yr_hip_graph_pack(const void* src, void* dst, int g, int rows, int cols, int dst_cols, const int64_t* strides6,
                      int dtype, void* stream);
/* dst[sum_d c_d dst_strides[d]] = src[sum_d c_d src_strides[d]] for every
 * coordinate c of dims (ndim <= 8; element strides, 0 broadcasts).  The tile
 * gathers and scatters of a customized op's input / output maps
 * (src/kernel/customized.cc, src/threadblock/input_loader.cc, output.cc) when
 * the op's threadblock graph runs operator by operator over all its tiles. */
int yr_hip_graph_copy_nd(const void* src, void* dst, int ndim, const int64_t* dims, const int64_t* src_strides,
                         const int64_t* dst_strides, int dtype, void* stream);
/* y = f(x) elementwise; kind 0 exp, 1 silu, 2 gelu (erf form), 3 relu,
 * 4 clamp(lo, hi), 5 sqrt, 6 square
 * (include/yirage/transpiler/runtime/kernel/element_unary.h:22-40), 7 x * lo
 * (the threadblock mul_scalar the reference's transpiler inserts for rms
 * accumulators, src/transpiler/transpile.cc:681-693). */
int yr_hip_graph_unary(const void* x, void* y, int64_t n, int kind, float lo, float hi, int dtype, void* stream);
/* out = a (op) b with size-1 broadcasting over ndim <= 6 dims (output dims
 * = elementwise max); kind 0 add, 1 mul, 2 div, 3 pow
 * (src/kernel/element_binary.cc:74-95). */
int yr_hip_graph_binary(const void* a, const void* b, void* out, int ndim, const int64_t* dims_a,
                        const int64_t* dims_b, int kind, int dtype, void* stream);
/* y[o][i] = sum_r x[o][r][i]: reduction(x, dim) to size 1
 * (src/kernel/reduction.cc:61-77, python reduction(A, dim) = size 1). */
int yr_hip_graph_reduction(const void* x, void* y, int64_t outer, int red, int64_t inner, int dtype, void* stream);
/* y[o][i] = max_r x[o][r][i] (threadblock reduction_max and the forloop
 * max accumulator, src/threadblock/reduction.cc, forloop_accum.cc:102-125). */
int yr_hip_graph_reduction_max(const void* x, void* y, int64_t outer, int red, int64_t inner, int dtype,
                               void* stream);
/* A tree of elementwise operators in one launch: y = program(x0..x_{n-1})
 * over the output dims (ndim <= 6; input k has dims in_dims[k][ndim], each 1
 * (broadcast) or the output's; all row-major dense).  prog[j] = {op, dst,
 * a, b, kind}: op 0 loads input a into register dst, 1 applies unary `kind`
 * (the yr_hip_graph_unary kinds; imm[2 j], imm[2 j + 1] = lo, hi) to
 * register a, 2 applies binary `kind` (yr_hip_graph_binary's) to registers
 * a, b; 16 registers, <= 32 instructions; y = the last instruction's
 * register.  Every result is rounded to dtype, so y is bit-identical to the
 * same operators run one launch each.  The fusion of single-consumer
 * elementwise chains of the reference's transpiler
 * (src/transpiler/resolve_tb_fusion.cc:35-66). */
int yr_hip_graph_ewise(const void* const* ins, int n, void* y, int ndim, const int64_t* out_dims,
                       const int64_t* in_dims, int n_prog, const int32_t* prog, const float* imm, int dtype,
                       void* stream);
/* One customized operator of a kernel graph in one launch: its threadblock
 * graph (src/threadblock/graph.cc; what the reference's transpiler turns
 * into generated CUDA, src/transpiler/transpile.cc:370-720) run as a tile
 * program, one workgroup per block of the grid (gx, gy, gz), every tile in
 * LDS as fp32, each operator's result rounded to dtype, accumulators fp32
 * over the forloop iterations.  program: int32 words (format in
 * csrc/tb_program.hip: header, tiles, inputs cut by input_map / forloop_dim
 * from dense row-major device tensors, operators, outputs placed by
 * output_map / forloop_dim); at most 800 words, 8 inputs, 4 outputs and
 * 160 KiB less 256 bytes of tiles.  The program is checked against the launch (every tile
 * and device access in bounds, operator shapes consistent) before anything
 * runs; YR_E_INVALID otherwise. */
int yr_hip_tb_program(const int32_t* program, int n_words, const void* const* ins, int n_in, void* const* outs,
                      int n_out, int gx, int gy, int gz, int dtype, void* stream);
/* The host-side check of yr_hip_tb_program alone (no device work): YR_OK
 * when the program would be accepted for that launch shape. */
int yr_hip_tb_program_check(const int32_t* program, int n_words, int n_in, int n_out, int gx, int gy, int gz);
/* y[row] = x[row] * rsqrt(mean(x[row]^2) + eps) over the n trailing
 * elements (rms_norm(X, normalized_shape), src/kernel/rms_norm.cc:71-114). */
int yr_hip_graph_rmsnorm(const void* x, void* y, int rows, int n, float eps, int dtype, void* stream);
/* c[b] = a[b] (m x k) @ b[b] (k x n), all row-major; n, k multiples of 8;
 * MFMA, fp32 accumulate (src/kernel/matmul.cc:44-96). */
int yr_hip_graph_matmul(const void* a, const void* b, void* c, int batch, int m, int n, int k, int dtype,
                        void* stream);

/* ------------------------------------------------------- generic launcher */
/* One operator by kind, with the shape of the reference's
 * execute_mugraph(inputs, outputs, buffer, stream, profiler) launcher
 * (python/yirage/kernel.py:22-72,411-421): inputs and outputs are arrays of
 * device pointers, `params` holds the integer shape/attribute list of the op
 * (floats travel as their IEEE-754 bits).  op_kind / layouts:
 *   YR_OP_RMSNORM_LINEAR: in {x, gamma|NULL, w}, out {o};
 *        params {batch, k, n, dtype, w_layout, eps_bits}
 *   YR_OP_GATED_MLP:      in {x, w1, w3}, out {o};
 *        params {batch, k, n, dtype, w_layout}
 *   YR_OP_GQA_PREFILL:    in {q, k, v}, out {o};
 *        params {batch, seq, hq, hkv, d, causal, dtype}
 *   YR_OP_LINEAR:         in {x, w, residual|NULL}, out {o};
 *        params {batch, k, n, dtype, w_layout}
 *   YR_OP_GQA_DECODE:     in {q, k_cache, v_cache, kv_indptr, kv_indices, kv_len}, out {o};
 *        params {batch, hq, hkv, d, page_size, max_kv_len, dtype}
 *   YR_OP_ATTENTION:      in {q, k, v}, out {o};
 *        params {G, M, L, d, dtype, scale_bits, strides12...}   (18 params)
 *   YR_OP_MATMUL:         in {a, b}, out {c}; params {batch, m, n, k, dtype}
 *   YR_OP_UNARY:          in {x}, out {y}; params {n, kind, dtype, lo_bits, hi_bits}
 *   YR_OP_BINARY:         in {a, b}, out {c}; params {ndim, kind, dtype, dims_a[ndim], dims_b[ndim]}
 *   YR_OP_REDUCTION:      in {x}, out {y}; params {outer, red, inner, dtype}
 *   YR_OP_RMSNORM:        in {x}, out {y}; params {rows, n, dtype, eps_bits}
 *   YR_OP_PACK:           in {src}, out {dst}; params {g, rows, cols, dst_cols, dtype, strides6...}
 *   YR_OP_COPY_ND:        in {src}, out {dst}; params {ndim, dtype, dims[8], src_strides[8], dst_strides[8],
 *                                             dst_offset[, src_offset]} (elements; 27 or 28 params)
 *   YR_OP_REDUCTION_MAX:  in {x}, out {y}; params {outer, red, inner, dtype}
 *   YR_OP_EWISE:          in {x0..x_{n-1}} (1..8), out {y}; params {ndim, n, n_prog, dtype,
 *                         out_dims[ndim], in_dims[n][ndim], prog[n_prog][5], imm_bits[n_prog][2]}
 *                         (see yr_hip_graph_ewise)
 *   YR_OP_TB_PROGRAM:     in {x0..} (1..8), out {y0..} (1..4); params {gx, gy, gz, dtype, program words...}
 *                         (see yr_hip_tb_program) */
#define YR_OP_RMSNORM_LINEAR 1
#define YR_OP_GATED_MLP 2
#define YR_OP_GQA_PREFILL 3
#define YR_OP_LINEAR 4
#define YR_OP_GQA_DECODE 5
#define YR_OP_ATTENTION 6
#define YR_OP_MATMUL 7
#define YR_OP_UNARY 8
#define YR_OP_BINARY 9
#define YR_OP_REDUCTION 10
#define YR_OP_RMSNORM 11
#define YR_OP_PACK 12
#define YR_OP_COPY_ND 13
#define YR_OP_REDUCTION_MAX 14
#define YR_OP_EWISE 15
#define YR_OP_TB_PROGRAM 16
int yr_hip_run_fused(int op_kind, int n_in, const void* const* inputs, int n_out, void* const* outputs,
                     int n_params, const int64_t* params, void* workspace, size_t workspace_bytes,
                     void* stream);
/* Workspace bytes yr_hip_run_fused needs for an op (0 if none); the
 * workspace layout is shared by every kind (tickets first), so one
 * zero-filled buffer of the maximum over a graph's steps serves them all. */
size_t yr_hip_fused_workspace(int op_kind, int n_params, const int64_t* params);

/* ------------------------------------------------------- persistent kernel */
/* Task graph of the persistent megakernel, built on the host (no GPU needed).
 * `json` describes the workers, tensors (name -> device pointer, dims,
 * dtype) and the ordered op list; see yirage_amd/persistent_kernel.py for the
 * producer.  Replaces Graph::generate_task_graph / register_mugraph /
 * sanity_check (src/kernel/runtime.cc:161-600,1416-1449). */
typedef struct yr_pk_graph yr_pk_graph;
typedef struct yr_pk_handle yr_pk_handle;
int yr_pk_graph_build(const char* json, yr_pk_graph** out);
void yr_pk_graph_free(yr_pk_graph* graph);
/* info[0..7] = ops, tasks, events, workers, tickets, scratch floats, longest queue, 0 */
int yr_pk_graph_info(const yr_pk_graph* graph, int64_t* info, int n);
/* rec[0..9] = op, task type, wait event, wait count, trigger event, row0, rows, i0, i1, i2 */
int yr_pk_graph_task(const yr_pk_graph* graph, int task, int64_t* rec, int n);
/* CPU replay of the queue/event protocol with random interleavings over
 * `epochs` launches, then (race_window > 0) a proof that every conflicting
 * tensor access pair within race_window ops is ordered.  YR_OK or
 * YR_E_GRAPH with the finding in `report`.  Mirrors sanity_check
 * (src/kernel/runtime.cc:540-600). */
int yr_pk_graph_simulate(const yr_pk_graph* graph, uint64_t seed, int epochs, int race_window, char* report,
                         size_t report_len);
/* The task graph in the reference's task_graph.json vocabulary
 * (all_tasks / all_events / first_tasks, runtime.cc:847-1318). */
int yr_pk_graph_export_json(const yr_pk_graph* graph, char* buf, size_t buf_len, size_t* needed);

/* Device pointers of the reference's meta tensors, in the order of
 * python/yirage/persistent_kernel.py:1291-1301. */
typedef struct {
  int32_t* step;
  int64_t* tokens;
  int64_t* input_tokens;
  int64_t* output_tokens;
  int32_t* num_new_tokens;
  int32_t* prompt_lengths;
  int32_t* qo_indptr;
  int32_t* paged_kv_indptr;
  int32_t* paged_kv_indices;
  int32_t* paged_kv_last_page_len;
} yr_pk_meta;

/* Uploads a built graph to the current device (cooperative launch of one
 * workgroup per worker).  Replaces init_persistent_kernel
 * (persistent_kernel.cuh:1036-1249); unlike it, state lives in the handle so
 * several persistent kernels can coexist. */
int yr_pk_create(const yr_pk_graph* graph, const yr_pk_meta* meta, yr_pk_handle** out);
/* Offline batch state (page queue, request slots) reset, as init_kernel
 * (persistent_kernel.cuh:107-132). */
int yr_pk_init_batch(yr_pk_handle* handle, void* stream);
/* Runs the task graph: up to max_iterations passes (decode / extend steps)
 * in one launch.  When the graph has a prepare_batch task, the device starts
 * the next pass only while that task left tokens to run, as the reference's
 * offline scheduler does on EVENT_END_OF_TASK_GRAPH
 * (persistent_kernel.cuh:841-857); max_iterations 0 then means "until every
 * request finished" (at most 2^20 passes).  Without a prepare_batch task
 * every pass runs (max_iterations >= 1 required).  Replaces
 * launch_persistent_kernel (persistent_kernel.cuh:1253-1318). */
int yr_pk_launch(yr_pk_handle* handle, void* stream, int max_iterations);
/* Synchronous read of the number of passes the last launch ran. */
int yr_pk_iterations(yr_pk_handle* handle, int* iterations);
/* Synchronous copy of the batch state the handle owns (the reference keeps
 * it in RuntimeConfig, persistent_kernel.cuh:107-132): request_ids
 * [max_requests], next_request_id, page_queue [max_pages], page_queue_head,
 * page_queue_tail, in that order (n >= max_requests + 3 + max_pages). */
int yr_pk_read_batch(yr_pk_handle* handle, int* out, size_t n);
/* 1 (default): cooperative launch.  0: ordinary launch of the same grid;
 * every worker was checked co-resident at create (occupancy x CUs >=
 * workers) and every wait stays under the watchdog.  For tools that do not
 * follow cooperative launches (profilers).  No reference counterpart. */
int yr_pk_set_launch_mode(yr_pk_handle* handle, int cooperative);
/* Batch > 1 graphs (max_num_batched_tokens > 1): copy every linear task's
 * weights into handle-owned memory in the order the task streams them
 * (16-row x 32-column MFMA fragments, 1 KiB per load instruction), so the
 * weight stream reads sequential 1 KiB units instead of 16 rows x 64 bytes.
 * enable 0 frees the copy and restores the original weight pointers.
 * `bytes` (optional) receives the size of the copy (about the linear
 * weights' size).  Synchronizes; not during a launch.  No reference
 * counterpart (a layout choice of this backend). */
int yr_pk_pack_weights(yr_pk_handle* handle, int enable, size_t* bytes);
/* Polls a dependency may spin before the watchdog flags an error (default
 * 2^26); the kernel then drains: every later wait gives up at once.  No
 * reference counterpart (its waits are unbounded). */
int yr_pk_set_spin_limit(yr_pk_handle* handle, long long polls);
/* Per-task timestamps (10 ns device clock) into buffer[task][8] =
 * {start, inputs ready, end, worker, s4, s5, s6, s7}; NULL disables.
 * GEMV tasks: s4 activations staged, s5 compute done, s6 outputs published.
 * Attention tasks: s5 request geometry read, s4 page ids read, s7 first K/V
 * block landed (profiling waits for it), s6 split merge done (merging task
 * only).  Replaces the
 * YPK_ENABLE_PROFILING ring buffer (persistent_kernel.cuh:473-480,608-635,
 * profiler.h:90-158). */
int yr_pk_set_profiler(yr_pk_handle* handle, uint64_t* buffer, size_t entries);
/* Synchronous read of the status words; YR_E_TIMEOUT after a watchdog exit. */
int yr_pk_status(yr_pk_handle* handle, int* status4);
/* After a watchdog exit (synchronizes): zero the status words, the event and
 * grid-barrier counters, the arrival tickets and every epoch-tagged word (link
 * tensors, split records), and restart the epochs. */
int yr_pk_reset_status(yr_pk_handle* handle);
/* Replaces finalize_persistent_kernel (persistent_kernel.cuh:1320-1363). */
void yr_pk_destroy(yr_pk_handle* handle);

/* ------------------------------------------------------- backend registry */
/* Restates BackendRegistry / BackendInterface
 * (include/yirage/backend/backend_registry.h:40-166,
 *  include/yirage/backend/backend_interface.h:40-212) with the `hip`
 * backend registered as BT_HIP.  Names/types follow
 * src/backend/backend_utils.cc:27-87 plus "hip". */
#define YR_BT_HIP 6
#define YR_BT_CPU 10
#define YR_BT_UNKNOWN 999
int yr_backend_num_registered(void);
/* writes the i-th registered backend name into buf; returns its type */
int yr_backend_registered_name(int i, char* buf, size_t buf_len);
int yr_backend_is_available(const char* name);
int yr_backend_type_from_name(const char* name);
/* default backend name by priority (hip first), "" if none available */
int yr_backend_default(char* buf, size_t buf_len);
/* BackendInterface::get_compile_flags() of a backend */
int yr_backend_compile_flags(const char* name, char* buf, size_t buf_len);

#ifdef __cplusplus
}
#endif

#endif /* YIRAGE_HIP_H_ */
