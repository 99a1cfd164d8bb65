// Task-graph records shared by the host builder (pk_builder.cc) and the
// persistent megakernel (pk_kernel.hip).  Plain PODs, identical layout on
// host and device.
//
// Restates the runtime ABI of include/yirage/persistent_kernel/
// runtime_header.h:47-269 (TaskDesc / EventDesc / RuntimeConfig) for this
// backend: a task carries one wait event and one trigger event; event
// counters are monotonic across launches (a wait is satisfied when the
// counter reaches num_triggers * epoch, as in the reference's
// num_triggers * iteration rule, persistent_kernel.cuh:582-604).
#pragma once
#include <stdint.h>

namespace yr {
namespace pk {

enum TaskType : int {
  TASK_NOP = 0,
  TASK_EMBED = 1,            // tasks/ampere/embedding.cuh:42-72
  TASK_LINEAR = 2,           // linear / linear_with_residual (linear_cutlass.cuh)
  TASK_RMSNORM_LINEAR = 3,   // rmsnorm (rmsnorm.cuh:76-128) fused into linear
  TASK_RMSNORM_LINEAR_SILU = 4,  // + silu_mul (silu_mul.cuh:31-40) on [gate | up] rows
  TASK_ATTENTION = 5,        // multitoken_paged_attention_4_16.cuh:40-656 (decode / short extend)
  TASK_RMSNORM_LINEAR_ARGMAX = 6,  // LM head + argmax_partial/reduce (argmax.cuh:71-155)
  TASK_PREPARE_BATCH = 7,    // prepare_next_batch (persistent_kernel.cuh:169-322)
};

enum OpFlags : int {
  OPF_RESIDUAL = 1,          // out = residual + x W^T
  OPF_X_LL = 2,              // x (qkv for attention) is a link tensor written by op x_src
  OPF_RES_LL = 4,            // residual is a link tensor written by op res_src
  OPF_OUT_LL = 8,            // out is a link tensor
  OPF_QK_NORM = 16,          // attention: per-head RMSNorm of q (weights `norm`) and new k (`k_norm`) before RoPE
  OPF_EMPTY_MERGER = 32,     // attention: the last split reads no cached positions (it appends and merges)
};

// Link tensors: activations passed between CUs inside one launch are stored
// as 8-byte words {bf16 pair (low 32 bits), tag (high 32 bits)}, one 64-bit
// store each (single-copy atomic).  tag = epoch << kLinkOpBits | producing op,
// so a reader accepts a word only if this launch's producer wrote it.
constexpr int kLinkOpBits = 10;
constexpr int kMaxLinkOps = 1 << kLinkOpBits;

// One per op (layer call).  Pointers are device addresses.
struct OpDesc {
  int type;
  int flags;
  int K;              // reduction dim (hidden / intermediate)
  int N;              // output columns of the whole op
  int x_ld, out_ld, res_ld;
  int max_tokens;     // rows of the activation buffers
  float eps;
  // attention
  int num_q_heads, num_kv_heads, head_dim, page_size, splits, qkv_ld;
  int ticket_base;    // first arrival ticket used by this op
  int vocab;          // argmax: valid columns (<= N)
  int scratch_off;    // float offset of this op's scratch records
  int x_src;          // op that wrote x (OPF_X_LL)
  int res_src;        // op that wrote the residual (OPF_RES_LL)
  int rec_rows;       // attention: query rows per split record (>= 16, max_tokens * G rounded up)
  const uint16_t* x;        // activations in
  const uint16_t* norm;     // RMSNorm weight
  uint16_t* out;            // activations out (column 0 of the op)
  const uint16_t* residual;
  uint16_t* k_cache;        // [pages][page][Hkv][D]
  uint16_t* v_cache;
  const uint16_t* cos_t;    // [pos][D]
  const uint16_t* sin_t;
  const int64_t* tokens_in; // embed: token ids [max_tokens]
  const uint16_t* table;    // embed: [vocab][hidden]
  int64_t* tokens_out;      // argmax: output token ids [max_tokens]
  const uint16_t* k_norm;   // attention qk-norm: k weights [head_dim] (q weights in `norm`)
  int attn_blocks;          // attention: cached 64-position blocks a split may read (7 waves x blocks per wave)
  int pad0;
};

// One per task (workgroup-sized unit of work).
struct TaskDesc {
  int op;             // index into OpDesc[]
  int wait_event;     // -1: none
  int wait_count;     // num_triggers of wait_event (per epoch)
  int trigger_event;  // -1: none
  int row0, rows;     // output rows / columns covered [row0, row0 + rows)
  int i0, i1;         // attention: request, kv head; argmax: task ordinal
  int i2, i3;         // attention: split index; argmax: number of tasks
  int split_row;      // linear: rows [0, split_row) come from w0, the rest from w1
  int packed;         // linear, batch > 1: w0 holds this task's weights in stream order (yr_pk_pack_weights)
  const uint16_t* w0; // weight rows of this task (gate rows for the SiLU op)
  const uint16_t* w1; // up rows for the SiLU op; second weight segment of a linear task
};

// Batch / page manager state (persistent_kernel.cuh:107-132,169-322).
struct BatchMeta {
  int* step;              // [total_requests]
  int64_t* tokens;        // [total_requests][max_seq_len]
  int64_t* input_tokens;  // [max_tokens]
  int64_t* output_tokens; // [max_tokens]
  int* num_new_tokens;    // [total_requests] (unused by offline mode)
  int* prompt_lengths;    // [total_requests]
  int* qo_indptr;         // [max_requests + 1]
  int* kv_indptr;         // [max_requests + 1]
  int* kv_indices;        // [max_pages]
  int* last_page_len;     // [max_requests]
  int* request_ids;       // [max_requests]
  int* next_request_id;   // [1]
  int* page_queue;        // [max_pages]
  int* page_queue_head;   // [1]
  int* page_queue_tail;   // [1]
  int* page_snap;         // [max_pages]: copy of kv_indices while prepare_batch rebuilds it
  int* status;            // [4]: [0] watchdog flag, [1] batch non-empty, [2] failing task, [3] spare
  int max_requests, max_tokens, max_pages, page_size, max_seq_len, total_requests;
  int online;             // online mode: prepare_batch advances step[0] by num_new_tokens[0] (host-fed)
  int64_t eos_token_id;
};

struct KernelArgs {
  const OpDesc* ops;
  const TaskDesc* tasks;
  const int* queue_offsets;  // [num_workers + 1]
  const int* queue;          // task ids, worker-major
  uint32_t* events;          // monotonic counters
  uint32_t* tickets;         // arrival tickets (zero at rest)
  float* scratch;            // split records
  BatchMeta meta;
  uint64_t* profile;         // optional [num_tasks][4]: start, inputs ready, end, worker
  uint32_t epoch;            // epoch of the launch's first task-graph pass (1, 2, 3, ...)
  int num_workers;
  long long spin_limit;      // watchdog: polls before a wait gives up
  // In-launch iteration (the reference's offline mode runs every step of a
  // generation in one launch, persistent_kernel.cuh:841-857): up to
  // max_iterations passes with epochs epoch, epoch + 1, ...; with
  // stop_when_empty the launch also ends after a pass whose prepare_batch
  // task left no tokens to run (status[1] == 0).
  int max_iterations;
  int stop_when_empty;
  uint32_t* grid_bar;        // grid barrier between passes: arrivals, +num_workers per barrier
  const uint32_t* event_triggers;  // [num events] num_triggers (epoch fast-forward after an early stop)
  int num_events;
  int* iterations_run;       // [1]: passes the last launch ran (written by worker 0)
};

}  // namespace pk
}  // namespace yr
