// Persistent megakernel for gfx950: one workgroup per CU runs its task queue;
// tasks wait on / trigger monotonic event counters; every task prefetches the
// bytes it can (weights, cached K/V) before it waits for its inputs.
//
// Replaces the reference runtime (include/yirage/persistent_kernel/
// persistent_kernel.cuh:454-974 worker/scheduler loops, 976-995 kernels,
// 1036-1363 entry points).  Differences by design:
//  * no scheduler warps: the host builds per-worker queues in topological op
//    order, so a worker only spins on the one event its next task needs;
//  * cross-XCD visibility without L2 maintenance: activations, split records
//    and tickets move with agent-scope (sc1) loads/stores, and a task's
//    completion is published with a relaxed agent-scope atomic after its
//    stores completed (vmcnt 0);
//  * a bounded spin (watchdog) turns a lost dependency into an error flag the
//    host reads back instead of a hang.
#include <string.h>

#include <vector>

#include "pk_builder.h"
#include "pk_types.h"
#include "yr_common.h"

namespace yr {
namespace pk {

constexpr int PK_WAVES = 8;
constexpr int PK_THREADS = PK_WAVES * kWave;
constexpr int XS_ELEMS = 32768;   // staged activation elements (64 KiB)
constexpr int OUT_ELEMS = 8192;   // staged task outputs (16 KiB)

struct Shared {
  uint16_t xs[XS_ELEMS];          // activations (bf16), [token][KB]
  uint16_t outs[OUT_ELEMS];       // task outputs (bf16), [token][rows]
  float red[PK_WAVES * 16 * 2];   // small reductions
  float attn_p[PK_WAVES][16][64]; // attention probabilities per wave
  float attn_ml[PK_WAVES][16][2];
  TaskDesc tq[256];               // this worker's first 256 task descriptors
  int flag;                       // last wait succeeded (0 after a watchdog exit)
  int last_op;                    // op whose activations are staged in xs (-1: none)
  int last_T;
};

// ------------------------------------------------------------ protocol
__device__ __forceinline__ bool aborted(const KernelArgs& a) {
  return __hip_atomic_load(a.meta.status, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) != 0;
}

// Whole-workgroup wait until events[e] >= wait_count * epoch.  Returns false
// when the watchdog fired here or elsewhere.
__device__ __forceinline__ uint64_t now_10ns() { return __builtin_amdgcn_s_memrealtime(); }

constexpr int POLL_T = (PK_WAVES - 1) * kWave;  // first lane of the sync wave (no weight loads)

__device__ bool wait_event(const KernelArgs& a, const TaskDesc& t, int task_id, Shared& sm) {
  if (t.wait_event < 0) {
    if (a.profile && threadIdx.x == POLL_T) a.profile[(size_t)task_id * 8 + 1] = now_10ns();
    return true;
  }
  if (threadIdx.x == POLL_T) {
    const uint32_t need = (uint32_t)t.wait_count * a.epoch;
    long long spins = 0;
    int ok = 1;
    for (;;) {
      uint32_t v = __hip_atomic_load(&a.events[t.wait_event], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      if ((int32_t)(v - need) >= 0) break;
      if ((spins & 255) == 255 && aborted(a)) { ok = 0; break; }
      if (++spins > a.spin_limit) {
        __hip_atomic_store(a.meta.status + 2, task_id, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        __hip_atomic_store(a.meta.status, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        ok = 0;
        break;
      }
      __builtin_amdgcn_s_sleep(2);
    }
    if (a.profile) a.profile[(size_t)task_id * 8 + 1] = now_10ns();
    sm.flag = ok;
  }
  __syncthreads();
  return sm.flag != 0;
}

// Publish completion: every thread's stores are complete, then one arrival.
__device__ void signal_event(const KernelArgs& a, const TaskDesc& t) {
  wait_vm();
  __syncthreads();
  if (threadIdx.x == POLL_T && t.trigger_event >= 0)
    __hip_atomic_fetch_add(&a.events[t.trigger_event], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

__device__ __forceinline__ uint32_t ld_agent_u32(const void* p) {
  return __hip_atomic_load(reinterpret_cast<const uint32_t*>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void st_agent_u32(void* p, uint32_t v) {
  __hip_atomic_store(reinterpret_cast<uint32_t*>(p), v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ uint4 ld_agent_u128(const void* p) {
  const uint64_t* q = reinterpret_cast<const uint64_t*>(p);
  uint64_t lo = __hip_atomic_load(q, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  uint64_t hi = __hip_atomic_load(q + 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  return make_uint4((uint32_t)lo, (uint32_t)(lo >> 32), (uint32_t)hi, (uint32_t)(hi >> 32));
}
__device__ __forceinline__ void st_agent_u128(void* p, uint4 v) {
  uint64_t* q = reinterpret_cast<uint64_t*>(p);
  __hip_atomic_store(q, (uint64_t)v.x | ((uint64_t)v.y << 32), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  __hip_atomic_store(q + 1, (uint64_t)v.z | ((uint64_t)v.w << 32), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

__device__ __forceinline__ int active_tokens(const KernelArgs& a, const OpDesc& op) {
  int n = (int)ld_agent_u32(a.meta.qo_indptr + a.meta.max_requests);
  return n < op.max_tokens ? n : op.max_tokens;
}

// ------------------------------------------------------------ embedding
__device__ void task_embed(const KernelArgs& a, const TaskDesc& t, int task_id, Shared& sm) {
  const OpDesc& op = a.ops[t.op];
  if (!wait_event(a, t, task_id, sm)) return;
  const int T = active_tokens(a, op);
  for (int b = 0; b < T; b++) {
    uint64_t tok = (uint64_t)__hip_atomic_load(reinterpret_cast<const uint64_t*>(op.tokens_in + b), __ATOMIC_RELAXED,
                                               __HIP_MEMORY_SCOPE_AGENT);
    if (tok >= (uint64_t)op.vocab) tok = 0;  // out-of-range ids read row 0
    const uint16_t* src = op.table + tok * (uint64_t)op.K + t.row0;
    uint16_t* dst = op.out + (size_t)b * op.out_ld + t.row0;
    for (int i = threadIdx.x * 8; i < t.rows; i += PK_THREADS * 8) st_agent_u128(dst + i, ldg16(src + i));
  }
  signal_event(a, t);
}

// ------------------------------------------------------------ GEMV family
// Workgroup roles: waves 0..CW-1 stream weights and do the dot products; the
// sync wave (wave CW) never loads weights, so its dependency polls and
// activation loads never wait (vmcnt is in order) behind weight traffic.
//   compute waves: issue stage 0 -> [X] -> stages (prefetch k+1, compute k)
//                  -> row sums to LDS -> [O]
//   sync wave:     poll the event -> stage activations (+RMSNorm) -> [X]
//                  -> [O] -> epilogue, stores, publish
// Between [O] of task i and [X] of task i+1 the compute waves already have
// task i+1's first stage in flight while the sync wave publishes task i and
// waits for task i+1's inputs.
enum { EPI_LIN = 0, EPI_NORM = 1, EPI_SILU = 2, EPI_ARGMAX = 3 };
constexpr int CW = PK_WAVES - 1;           // compute waves
constexpr int SYNC_T0 = CW * kWave;        // first thread of the sync wave

// A stage holds NM x RI rows x NCH chunks of 16 bytes per lane (NM*RI*NCH = 8
// loads): a sub-block of SB = NCH * 512 elements of every row in the stage.
// Eight loads per lane keep ~57 KB per CU in flight, about bandwidth x
// latency; deeper prefetch only lengthens the CU's memory queue in front of
// the latency-critical polls and activation loads.
template <int NM, int RI, int NCH>
struct Stage {
  uint4 w[NM][RI][NCH];
};

template <int NM, int RI, int NCH>
__device__ __forceinline__ void load_stage(Stage<NM, RI, NCH>& s, const TaskDesc& t, int K, int wave, int lane,
                                           int group, int sb, int R) {
#pragma unroll
  for (int m = 0; m < NM; m++) {
#pragma unroll
    for (int r = 0; r < RI; r++) {
      int row = wave + CW * (group * RI + r);
      // SiLU op: matrix m = gate / up; linear op: row split across two segments
      const uint16_t* W;
      if (NM == 2) W = (m == 0 ? t.w0 : t.w1) + (size_t)row * K;
      else W = row < t.split_row ? t.w0 + (size_t)row * K : t.w1 + (size_t)(row - t.split_row) * K;
#pragma unroll
      for (int j = 0; j < NCH; j++) {
        int k = sb * (NCH * 512) + (lane + 64 * j) * 8;
        if (row < R && k < K) s.w[m][r][j] = ldg16(W + k);
        else s.w[m][r][j] = make_uint4(0, 0, 0, 0);
      }
    }
  }
}

template <int TM, int NM, int RI, int NCH>
__device__ __forceinline__ void compute_stage(const Stage<NM, RI, NCH>& s, const Shared& sm, int KB, int kb_off,
                                              int sb, int K, int lane, float (&acc)[NM][RI][TM]) {
#pragma unroll
  for (int j = 0; j < NCH; j++) {
    int kl = sb * (NCH * 512) + (lane + 64 * j) * 8 - kb_off;  // element offset inside the staged block
    if (kb_off + kl >= K) continue;
    uint4 xv[TM];
#pragma unroll
    for (int b = 0; b < TM; b++) xv[b] = *reinterpret_cast<const uint4*>(&sm.xs[b * KB + kl]);
#pragma unroll
    for (int m = 0; m < NM; m++)
#pragma unroll
      for (int r = 0; r < RI; r++) {
        const uint4 w = s.w[m][r][j];
#pragma unroll
        for (int b = 0; b < TM; b++) {
          float v = acc[m][r][b];
          v = dot2<DT_BF16>(w.x, xv[b].x, v);
          v = dot2<DT_BF16>(w.y, xv[b].y, v);
          v = dot2<DT_BF16>(w.z, xv[b].z, v);
          v = dot2<DT_BF16>(w.w, xv[b].w, v);
          acc[m][r][b] = v;
        }
      }
  }
}

// Sync wave: activations [T][kb_off .. kb_off + KB) into LDS (agent-scope
// loads, 16 per lane in flight), RMSNorm applied when NORM
// (x * (rsqrt(mean(x^2) + eps) * w), rounded to bf16 as rmsnorm.cuh:120-124).
// RMSNorm weights of one sync-wave lane (K <= 4096): loaded before the poll,
// since they never depend on the event.
struct NormRegs {
  uint4 g[8];
};

__device__ __forceinline__ void load_norm(NormRegs& nr, const OpDesc& op, int lane) {
#pragma unroll
  for (int j = 0; j < 8; j++) {
    int c = (lane + kWave * j) * 8;
    nr.g[j] = c < op.K ? ldg16(op.norm + c) : make_uint4(0, 0, 0, 0);
  }
}

template <int TM, bool NORM>
__device__ __forceinline__ void stage_x_sync(const OpDesc& op, int T, int KB, int kb_off, Shared& sm, const NormRegs& nr,
                                             bool have_nr) {
  const int lane = threadIdx.x - SYNC_T0;
  const int K = op.K;
  const int n8 = KB / 8;
  const int total = TM * n8;
  for (int i0 = 0; i0 < total; i0 += kWave * 16) {
    uint4 v[16];
#pragma unroll
    for (int u = 0; u < 16; u++) {
      int i = i0 + u * kWave + lane;
      int b = i / n8, c = (i % n8) * 8;
      v[u] = (i < total && b < T && kb_off + c < K) ? ld_agent_u128(op.x + (size_t)b * op.x_ld + kb_off + c)
                                                     : make_uint4(0, 0, 0, 0);
    }
#pragma unroll
    for (int u = 0; u < 16; u++) {
      int i = i0 + u * kWave + lane;
      if (i < total) *reinterpret_cast<uint4*>(&sm.xs[(i / n8) * KB + (i % n8) * 8]) = v[u];
    }
  }
  if constexpr (NORM) {
    // K <= KB here (checked at build): one pass per token
    for (int b = 0; b < TM; b++) {
      float ss = 0.f;
      for (int c = lane * 8; c < K; c += kWave * 8) {
        uint4 v = *reinterpret_cast<const uint4*>(&sm.xs[b * KB + c]);
        uint32_t w4[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
        for (int e = 0; e < 4; e++) {
          float lo = lo16<DT_BF16>(w4[e]), hi = hi16<DT_BF16>(w4[e]);
          ss += lo * lo + hi * hi;
        }
      }
      ss = wave_sum(ss);
      float r = rsqrtf(ss / (float)K + op.eps);
      if (b >= T) continue;
      auto norm_chunk = [&](int c, uint4 g) __attribute__((always_inline)) {
        uint4 v = *reinterpret_cast<const uint4*>(&sm.xs[b * KB + c]);
        uint32_t xv[4] = {v.x, v.y, v.z, v.w}, gv[4] = {g.x, g.y, g.z, g.w}, o[4];
#pragma unroll
        for (int e = 0; e < 4; e++) {
          float lo = lo16<DT_BF16>(xv[e]) * (r * lo16<DT_BF16>(gv[e]));
          float hi = hi16<DT_BF16>(xv[e]) * (r * hi16<DT_BF16>(gv[e]));
          o[e] = pack2<DT_BF16>(lo, hi);
        }
        *reinterpret_cast<uint4*>(&sm.xs[b * KB + c]) = make_uint4(o[0], o[1], o[2], o[3]);
      };
      if (have_nr) {
#pragma unroll
        for (int j = 0; j < 8; j++) {
          int c = (lane + kWave * j) * 8;
          if (c < K) norm_chunk(c, nr.g[j]);
        }
      } else {
        for (int c = lane * 8; c < K; c += kWave * 8) norm_chunk(c, ldg16(op.norm + c));
      }
    }
  }
}

// Sync wave: one-lane event poll (the watchdog exits through sm.flag).
__device__ bool poll_event_sync(const KernelArgs& a, const TaskDesc& t, int task_id, Shared& sm) {
  if (threadIdx.x == SYNC_T0) {
    int ok = 1;
    if (t.wait_event >= 0) {
      const uint32_t need = (uint32_t)t.wait_count * a.epoch;
      long long spins = 0;
      for (;;) {
        uint32_t v = __hip_atomic_load(&a.events[t.wait_event], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        if ((int32_t)(v - need) >= 0) break;
        if ((spins & 255) == 255 && aborted(a)) { ok = 0; break; }
        if (++spins > a.spin_limit) {
          __hip_atomic_store(a.meta.status + 2, task_id, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
          __hip_atomic_store(a.meta.status, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
          ok = 0;
          break;
        }
        __builtin_amdgcn_s_sleep(2);
      }
    }
    if (a.profile) a.profile[(size_t)task_id * 8 + 1] = now_10ns();
    sm.flag = ok;
  }
  __builtin_amdgcn_wave_barrier();
  return __shfl(sm.flag, 0, kWave) != 0;
}

template <int TM, int EPI>
__device__ void task_gemv(const KernelArgs& a, const TaskDesc& t, int task_id, Shared& sm) {
  constexpr int NM = EPI == EPI_SILU ? 2 : 1;
  constexpr int RI = 1;
  constexpr int NCH = 8 / NM;          // chunks per lane per matrix per stage
  constexpr int SB = NCH * 512;        // elements per sub-block
  constexpr bool NORM = EPI != EPI_LIN;
  const OpDesc& op = a.ops[t.op];
  const int K = op.K, R = t.rows;
  // wave index as a scalar: role branches are wave-uniform, so the register
  // live ranges of the sync and compute paths do not overlap
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave), lane = threadIdx.x % kWave;
  const bool is_sync = wave == CW;
  const int KB = TM == 1 ? K : (K < 4096 ? K : 4096);   // staged activation block
  const int nkb = (K + KB - 1) / KB;
  const int nsb = (KB + SB - 1) / SB;                     // sub-blocks per staged block
  float* outs = reinterpret_cast<float*>(sm.outs);       // [T][R] fp32 row sums (SiLU: products)
  const bool same_op = sm.last_op == t.op && nkb == 1;   // inputs of this op already staged

  if (is_sync) {
    // ---------------- sync wave: inputs
    int T = sm.last_T;
    if (!same_op) {
      NormRegs nr;
      const bool pre = NORM && K <= 4096;
      if (pre) load_norm(nr, op, lane);
      bool ok = poll_event_sync(a, t, task_id, sm);
      if (ok) {
        T = active_tokens(a, op);
        stage_x_sync<TM, NORM>(op, T, KB, 0, sm, nr, pre);
      }
    } else if (a.profile && lane == 0) {
      a.profile[(size_t)task_id * 8 + 1] = now_10ns();
    }
    if (lane == 0) {
      sm.last_T = T;
      sm.last_op = nkb == 1 ? t.op : -1;
    }
  }
  // compute waves: first stage in flight before the inputs are ready
  const int nrows_w = (!is_sync && wave < R) ? (R - wave + CW - 1) / CW : 0;
  const int ngroups = (nrows_w + RI - 1) / RI;
  Stage<NM, RI, NCH> cur, nxt;
  if (ngroups > 0) load_stage<NM, RI, NCH>(cur, t, K, wave, lane, 0, 0, R);
  __syncthreads();  // [X]: activations block 0 staged
  if (a.profile && threadIdx.x == SYNC_T0) a.profile[(size_t)task_id * 8 + 4] = now_10ns();
  if (!sm.flag) return;
  const int T = sm.last_T;

  // row groups kept live across staged blocks: only a plain linear can have
  // K > KB (RMSNorm ops stage all of K, the builder checks it)
  constexpr int GMAX = NORM ? 1 : 3;
  float acc_keep[GMAX][NM][RI][TM];
#pragma unroll
  for (int g = 0; g < GMAX; g++)
#pragma unroll
    for (int m = 0; m < NM; m++)
#pragma unroll
      for (int r = 0; r < RI; r++)
#pragma unroll
        for (int b = 0; b < TM; b++) acc_keep[g][m][r][b] = 0.f;

  auto finish_group = [&](int g, float (&acc)[NM][RI][TM]) __attribute__((always_inline)) {
#pragma unroll
    for (int r = 0; r < RI; r++) {
      int row = wave + CW * (g * RI + r);
#pragma unroll
      for (int b = 0; b < TM; b++) {
        float v0 = wave_sum(acc[0][r][b]);
        float v1 = NM == 2 ? wave_sum(acc[NM - 1][r][b]) : 0.f;
        if (lane == 0 && row < R && b < T) {
          float o = v0;
          if constexpr (EPI == EPI_SILU) {
            // silu_mul.cuh:31-40 on the bf16 gate/up results
            float gt = round_to<DT_BF16>(v0), up = round_to<DT_BF16>(v1);
            o = round_to<DT_BF16>(gt / (1.0f + expf(-gt))) * up;
          }
          outs[b * R + row] = o;
        }
      }
    }
  };

  for (int kb = 0; kb < nkb; kb++) {
    if (kb) {
      __syncthreads();  // compute waves are done with block kb-1
      if (is_sync) {
        NormRegs none;
        stage_x_sync<TM, false>(op, T, KB, kb * KB, sm, none, false);
      }
      __syncthreads();  // block kb staged
    }
    if (is_sync) continue;
    const int nst = ngroups * nsb;
    for (int st = 0; st < nst; st++) {
      int g = st / nsb, sb = kb * nsb + st % nsb;
      int st2 = st + 1, kb2 = kb;
      if (st2 == nst) { st2 = 0; kb2 = kb + 1; }
      bool has_next = kb2 < nkb && ngroups > 0;
      if (has_next) load_stage<NM, RI, NCH>(nxt, t, K, wave, lane, st2 / nsb, kb2 * nsb + st2 % nsb, R);
      float acc[NM][RI][TM];
      if (nkb > 1) {
#pragma unroll
        for (int gg = 0; gg < GMAX; gg++)
          if (gg == g)
#pragma unroll
            for (int m = 0; m < NM; m++)
#pragma unroll
              for (int r = 0; r < RI; r++)
#pragma unroll
                for (int b = 0; b < TM; b++) acc[m][r][b] = acc_keep[gg][m][r][b];
      } else if (st % nsb == 0) {
#pragma unroll
        for (int m = 0; m < NM; m++)
#pragma unroll
          for (int r = 0; r < RI; r++)
#pragma unroll
            for (int b = 0; b < TM; b++) acc[m][r][b] = 0.f;
      } else {
#pragma unroll
        for (int m = 0; m < NM; m++)
#pragma unroll
          for (int r = 0; r < RI; r++)
#pragma unroll
            for (int b = 0; b < TM; b++) acc[m][r][b] = acc_keep[0][m][r][b];
      }
      compute_stage<TM, NM, RI, NCH>(cur, sm, KB, kb * KB, sb, K, lane, acc);
      bool last_sb = st % nsb == nsb - 1;
      if (nkb > 1) {
#pragma unroll
        for (int gg = 0; gg < GMAX; gg++)
          if (gg == g)
#pragma unroll
            for (int m = 0; m < NM; m++)
#pragma unroll
              for (int r = 0; r < RI; r++)
#pragma unroll
                for (int b = 0; b < TM; b++) acc_keep[gg][m][r][b] = acc[m][r][b];
        if (kb == nkb - 1 && last_sb) finish_group(g, acc);
      } else if (last_sb) {
        finish_group(g, acc);
      } else {
#pragma unroll
        for (int m = 0; m < NM; m++)
#pragma unroll
          for (int r = 0; r < RI; r++)
#pragma unroll
            for (int b = 0; b < TM; b++) acc_keep[0][m][r][b] = acc[m][r][b];
      }
      if (has_next) cur = nxt;
    }
  }
  __syncthreads();  // [O]: row sums of every compute wave are in LDS
  if (a.profile && threadIdx.x == SYNC_T0) a.profile[(size_t)task_id * 8 + 5] = now_10ns();
  if (!is_sync) return;

  // ---------------- sync wave: epilogue, stores, publish
  for (int i = lane; i < T * (R / 2); i += kWave) {
    int b = i / (R / 2), p = i % (R / 2);
    float v0 = outs[b * R + 2 * p], v1 = outs[b * R + 2 * p + 1];
    if (EPI != EPI_SILU && (op.flags & OPF_RESIDUAL)) {
      uint32_t rw = ld_agent_u32(op.residual + (size_t)b * op.res_ld + t.row0 + 2 * p);
      v0 += lo16<DT_BF16>(rw);
      v1 += hi16<DT_BF16>(rw);
    }
    uint32_t packed = pack2<DT_BF16>(v0, v1);
    st_agent_u32(op.out + (size_t)b * op.out_ld + t.row0 + 2 * p, packed);
    if (EPI == EPI_ARGMAX) {
      outs[b * R + 2 * p] = lo16<DT_BF16>(packed);  // argmax runs on the bf16 logits
      outs[b * R + 2 * p + 1] = hi16<DT_BF16>(packed);
    }
  }
  if constexpr (EPI == EPI_ARGMAX) {
    // local (value, index) maximum per token over this task's valid rows;
    // lowest index wins ties (torch.argmax semantics)
    __builtin_amdgcn_wave_barrier();
    const int lim = op.vocab - t.row0 < R ? op.vocab - t.row0 : R;
    for (int b = 0; b < T; b++) {
      float best = -INFINITY;
      int bi = 0x7fffffff;
      for (int i = lane; i < lim; i += kWave) {
        float v = outs[b * R + i];
        if (v > best || (v == best && i < bi)) { best = v; bi = i; }
      }
#pragma unroll
      for (int o = 32; o > 0; o >>= 1) {
        float ov = __shfl_xor(best, o, kWave);
        int oi = __shfl_xor(bi, o, kWave);
        if (ov > best || (ov == best && oi < bi)) { best = ov; bi = oi; }
      }
      if (lane == 0) {
        float* rec = a.scratch + op.scratch_off + ((size_t)t.i0 * op.max_tokens + b) * 2;
        st_agent(rec, best);
        st_agent(rec + 1, __int_as_float(bi == 0x7fffffff ? -1 : t.row0 + bi));
      }
    }
    wait_vm();
    int last = 0;
    if (lane == 0)
      last = __hip_atomic_fetch_add(&a.tickets[op.ticket_base], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) ==
             (uint32_t)(t.i1 - 1);
    last = __shfl(last, 0, kWave);
    if (last) {
      if (lane == 0) __hip_atomic_store(&a.tickets[op.ticket_base], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      // reduce every task's record; task order = column order
      for (int b = 0; b < T; b++) {
        float best = -INFINITY;
        int bi = 0x7fffffff;
        for (int k = lane; k < t.i1; k += kWave) {
          const float* rec = a.scratch + op.scratch_off + ((size_t)k * op.max_tokens + b) * 2;
          float v = ld_agent(rec);
          int idx = __float_as_int(ld_agent(rec + 1));
          if (idx >= 0 && (v > best || (v == best && idx < bi))) { best = v; bi = idx; }
        }
#pragma unroll
        for (int o = 32; o > 0; o >>= 1) {
          float ov = __shfl_xor(best, o, kWave);
          int oi = __shfl_xor(bi, o, kWave);
          if (ov > best || (ov == best && oi < bi)) { best = ov; bi = oi; }
        }
        if (lane == 0)
          __hip_atomic_store(reinterpret_cast<uint64_t*>(op.tokens_out + b),
                             (uint64_t)(int64_t)(bi == 0x7fffffff ? -1 : bi), __ATOMIC_RELAXED,
                             __HIP_MEMORY_SCOPE_AGENT);
      }
    }
  }
  wait_vm();
  if (a.profile && lane == 0) a.profile[(size_t)task_id * 8 + 6] = now_10ns();
  if (lane == 0 && t.trigger_event >= 0)
    __hip_atomic_fetch_add(&a.events[t.trigger_event], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// ------------------------------------------------------------ attention
// One task = (request r, kv head h, split s).  Cached positions [0, base) are
// divided between the splits; the last split also handles the new tokens
// (RoPE, append to the paged cache, causal mask), as the reference does in
// multitoken_paged_attention_4_16.cuh:227-560.  Query rows = token j * G + g
// (<= 16) in one MFMA 16x16x32 row block.
__device__ __forceinline__ f32x4 mfma_bf16(uint4 a, uint4 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8v, a), __builtin_bit_cast(bf16x8v, b), c,
                                                 0, 0, 0);
}

// RoPE (rotate-half, rotary_embedding.cuh:22-81) of elements d .. d+7 of one
// head vector `src` at position pos, rounded to bf16, packed.
__device__ __forceinline__ uint4 rope8(const uint16_t* src, int d, int D, const OpDesc& op, int pos) {
  uint4 x = ld_agent_u128(src + d);
  if (!op.cos_t) return x;
  int half = D / 2;
  int dp = d < half ? d + half : d - half;
  uint4 y = ld_agent_u128(src + dp);
  uint4 c = ldg16(op.cos_t + (size_t)pos * D + d), s = ldg16(op.sin_t + (size_t)pos * D + d);
  uint32_t xv[4] = {x.x, x.y, x.z, x.w}, yv[4] = {y.x, y.y, y.z, y.w}, cv[4] = {c.x, c.y, c.z, c.w},
           sv[4] = {s.x, s.y, s.z, s.w}, o[4];
  float sg = d < half ? -1.f : 1.f;
#pragma unroll
  for (int e = 0; e < 4; e++) {
    float lo = lo16<DT_BF16>(xv[e]) * lo16<DT_BF16>(cv[e]) + sg * lo16<DT_BF16>(yv[e]) * lo16<DT_BF16>(sv[e]);
    float hi = hi16<DT_BF16>(xv[e]) * hi16<DT_BF16>(cv[e]) + sg * hi16<DT_BF16>(yv[e]) * hi16<DT_BF16>(sv[e]);
    o[e] = pack2<DT_BF16>(lo, hi);
  }
  return make_uint4(o[0], o[1], o[2], o[3]);
}

template <int RMAX>
__device__ void task_attention(const KernelArgs& a, const TaskDesc& t, int task_id, Shared& sm) {
  const OpDesc& op = a.ops[t.op];
  constexpr int D = 128;
  const int r = t.i0, h = t.i1, s = t.i2, S = op.splits;
  const int G = op.num_q_heads / op.num_kv_heads;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave), lane = threadIdx.x % kWave;
  const BatchMeta& m = a.meta;
  // request geometry (the page table is written by the host or by the
  // previous launch's prepare_batch task)
  const int t0 = m.qo_indptr[r], nt = m.qo_indptr[r + 1] - t0;
  const int pb = m.kv_indptr[r], np = m.kv_indptr[r + 1] - pb;
  const int lpl = m.last_page_len[r];
  const int seq = nt > 0 ? (np - 1) * op.page_size + (lpl == 0 ? op.page_size : lpl) : 0;
  const int base = seq - nt;
  int chunk = (base + S - 1) / S;
  chunk = (chunk + 15) & ~15;
  const int c0 = s * chunk < base ? s * chunk : base;
  const int c1 = (s + 1) * chunk < base ? (s + 1) * chunk : base;
  const bool last = s == S - 1;
  const size_t tok_stride = (size_t)op.num_kv_heads * D;
  auto cache_off = [&](int pos) __attribute__((always_inline)) -> size_t {
    int pg = m.kv_indices[pb + pos / op.page_size];
    return ((size_t)pg * op.page_size + pos % op.page_size) * tok_stride + (size_t)h * D;
  };
  const float scale = 1.4426950408889634f / sqrtf((float)D);

  // cached positions: blocks of 64 per wave (wave w: blocks w, w + 8, ...)
  const int nblk = (c1 - c0 + 63) / 64;
  // prefetch the first block of this wave before waiting
  uint4 kf[4][4], vf[16];
  auto load_block = [&](int blk) __attribute__((always_inline)) {
    int p0 = c0 + blk * 64;
#pragma unroll
    for (int j = 0; j < 4; j++) {
      int p = p0 + 16 * j + lane % 16;
      bool ok = p < c1;
      size_t off = ok ? cache_off(p) : 0;
#pragma unroll
      for (int q = 0; q < 4; q++) kf[j][q] = ok ? ldg16(op.k_cache + off + 32 * q + (lane / 16) * 8) : make_uint4(0, 0, 0, 0);
    }
#pragma unroll
    for (int i = 0; i < 16; i++) {
      int p = p0 + lane / 16 + 4 * i;
      vf[i] = p < c1 ? ldg16(op.v_cache + cache_off(p) + (lane % 16) * 8) : make_uint4(0, 0, 0, 0);
    }
  };
  if (nt > 0 && wave < nblk && wave < CW) load_block(wave);

  if (!wait_event(a, t, task_id, sm)) return;
  if (nt <= 0) {
    signal_event(a, t);
    return;
  }
  if (nt * G > 16 || nblk > CW) {  // beyond one MFMA row block / one block per wave
    if (threadIdx.x == 0) {
      __hip_atomic_store(a.meta.status + 3, task_id + 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    signal_event(a, t);
    return;
  }
  const uint16_t* qkv = op.x + (size_t)t0 * op.qkv_ld + (size_t)h * (G + 2) * D;

  // Q fragments: row = j * G + g, k = d
  uint4 qf[4];
  {
    int row = lane % 16, j = row / G, g = row % G;
    bool ok = row < nt * G;
#pragma unroll
    for (int q = 0; q < 4; q++)
      qf[q] = ok ? rope8(qkv + (size_t)j * op.qkv_ld + (size_t)g * D, 32 * q + (lane / 16) * 8, D, op, base + j)
                 : make_uint4(0, 0, 0, 0);
  }

  // per-wave online softmax state for rows 4*(lane/16)+i
  float m_i[4], l_i[4];
  float o_acc[RMAX][8];  // [query row][8 dims of this lane's d-chunk]
#pragma unroll
  for (int i = 0; i < 4; i++) { m_i[i] = -INFINITY; l_i[i] = 0.f; }
#pragma unroll
  for (int rr = 0; rr < RMAX; rr++)
#pragma unroll
    for (int e = 0; e < 8; e++) o_acc[rr][e] = 0.f;

  // process one 64-position block held in kf/vf; mask(p_local, row) -> visible
  auto process = [&](int p0, int npos, bool causal_new) __attribute__((always_inline)) {
    f32x4 sc[4];
#pragma unroll
    for (int j = 0; j < 4; j++) {
      f32x4 c = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int q = 0; q < 4; q++) c = mfma_bf16(qf[q], kf[j][q], c);
      sc[j] = c;
    }
#pragma unroll
    for (int i = 0; i < 4; i++) {
      int row = 4 * (lane / 16) + i;
      int tj = row / G;
      float mx = -INFINITY;
#pragma unroll
      for (int j = 0; j < 4; j++) {
        int pl = 16 * j + lane % 16;
        bool ok = pl < npos && row < nt * G && (!causal_new || pl <= tj);
        float v = ok ? sc[j][i] * scale : -INFINITY;
        sc[j][i] = v;
        mx = fmaxf(mx, v);
      }
#pragma unroll
      for (int o = 8; o > 0; o >>= 1) mx = fmaxf(mx, __shfl_xor(mx, o, kWave));
      float mnew = fmaxf(m_i[i], mx);
      float alpha = mnew == -INFINITY ? 1.f : exp2f(m_i[i] - mnew);
      float ls = 0.f;
#pragma unroll
      for (int j = 0; j < 4; j++) {
        float p = mnew == -INFINITY ? 0.f : exp2f(sc[j][i] - mnew);
        ls += p;
        sm.attn_p[wave][row][16 * j + lane % 16] = p;
      }
#pragma unroll
      for (int o = 8; o > 0; o >>= 1) ls += __shfl_xor(ls, o, kWave);
      l_i[i] = l_i[i] * alpha + ls;
      m_i[i] = mnew;
      if ((lane % 16) == 0) sm.attn_ml[wave][row][0] = alpha;
    }
    __builtin_amdgcn_s_waitcnt(0xc07f);
    __builtin_amdgcn_wave_barrier();
    // O[row][d] = O * alpha + sum_p P[row][p] V[p][d]; lane: d-chunk lane%16, positions lane/16 + 4i
#pragma unroll
    for (int rr = 0; rr < RMAX; rr++) {
      float al = sm.attn_ml[wave][rr][0];
#pragma unroll
      for (int e = 0; e < 8; e++) o_acc[rr][e] *= al;
    }
#pragma unroll
    for (int i = 0; i < 16; i++) {
      int pl = lane / 16 + 4 * i;
      uint32_t vw[4] = {vf[i].x, vf[i].y, vf[i].z, vf[i].w};
      float v[8];
#pragma unroll
      for (int e = 0; e < 4; e++) {
        v[2 * e] = lo16<DT_BF16>(vw[e]);
        v[2 * e + 1] = hi16<DT_BF16>(vw[e]);
      }
#pragma unroll
      for (int rr = 0; rr < RMAX; rr++) {
        float p = sm.attn_p[wave][rr][pl];
#pragma unroll
        for (int e = 0; e < 8; e++) o_acc[rr][e] = fmaf(p, v[e], o_acc[rr][e]);
      }
    }
    __builtin_amdgcn_wave_barrier();
  };

  // one 64-position block per compute wave (the builder sizes splits so that
  // a split never holds more than CW * 64 cached positions)
  if (wave < nblk && wave < CW) process(c0 + wave * 64, (c1 - c0) - wave * 64 < 64 ? (c1 - c0) - wave * 64 : 64, false);

  // new tokens (last split, wave 0): k/v from qkv, RoPE on k, append to cache
  if (last && wave == 0) {
#pragma unroll
    for (int j = 0; j < 4; j++) {
      int i = 16 * j + lane % 16;
      bool ok = j == 0 && i < nt;
#pragma unroll
      for (int q = 0; q < 4; q++) {
        int d = 32 * q + (lane / 16) * 8;
        uint4 kv = ok ? rope8(qkv + (size_t)i * op.qkv_ld + (size_t)G * D, d, D, op, base + i) : make_uint4(0, 0, 0, 0);
        kf[j][q] = kv;
        if (ok) *reinterpret_cast<uint4*>(op.k_cache + cache_off(base + i) + d) = kv;
      }
    }
#pragma unroll
    for (int i2 = 0; i2 < 16; i2++) {
      int i = lane / 16 + 4 * i2;
      bool ok = i < nt;
      uint4 vv = ok ? ld_agent_u128(qkv + (size_t)i * op.qkv_ld + (size_t)(G + 1) * D + (lane % 16) * 8)
                    : make_uint4(0, 0, 0, 0);
      vf[i2] = vv;
      if (ok) *reinterpret_cast<uint4*>(op.v_cache + cache_off(base + i) + (lane % 16) * 8) = vv;
    }
    process(base, nt, true);
  }

  // sum o over the 4 lane groups (positions lane/16 + 4 i), then merge the
  // 8 waves: per row, (m, l) in LDS, o through LDS (xs reused as float)
#pragma unroll
  for (int rr = 0; rr < RMAX; rr++)
#pragma unroll
    for (int e = 0; e < 8; e++) {
      float x = o_acc[rr][e];
      x += __shfl_xor(x, 16, kWave);
      x += __shfl_xor(x, 32, kWave);
      o_acc[rr][e] = x;
    }
  float* o_lds = reinterpret_cast<float*>(sm.xs);  // [wave][16 rows][128]
  __syncthreads();
  if (lane < 16) {
#pragma unroll
    for (int rr = 0; rr < RMAX; rr++)
#pragma unroll
      for (int e = 0; e < 8; e++) o_lds[(wave * 16 + rr) * D + lane * 8 + e] = o_acc[rr][e];
  }
  // lanes 16*(i)..: row 4*(lane/16)+i holds m_i/l_i
  if ((lane % 16) == 0) {
#pragma unroll
    for (int i = 0; i < 4; i++) {
      sm.attn_ml[wave][4 * (lane / 16) + i][0] = m_i[i];
      sm.attn_ml[wave][4 * (lane / 16) + i][1] = l_i[i];
    }
  }
  __syncthreads();
  const int rows = nt * G;
  float* rec_base = a.scratch + op.scratch_off + (((size_t)r * op.num_kv_heads + h) * S) * kAttnRecFloats;
  float* rec = rec_base + (size_t)s * kAttnRecFloats;
  for (int idx = threadIdx.x; idx < rows * D; idx += PK_THREADS) {
    int rr = idx / D, d = idx % D;
    float M = -INFINITY;
#pragma unroll
    for (int w = 0; w < PK_WAVES; w++) M = fmaxf(M, sm.attn_ml[w][rr][0]);
    float L = 0.f, O = 0.f;
#pragma unroll
    for (int w = 0; w < PK_WAVES; w++) {
      float f = sm.attn_ml[w][rr][0] == -INFINITY ? 0.f : exp2f(sm.attn_ml[w][rr][0] - M);
      L += sm.attn_ml[w][rr][1] * f;
      O += o_lds[(w * 16 + rr) * D + d] * f;
    }
    st_agent(rec + rr * (D + 2) + d, O);
    if (d == 0) {
      st_agent(rec + rr * (D + 2) + D, M);
      st_agent(rec + rr * (D + 2) + D + 1, L);
    }
  }
  if (arrive_last(&a.tickets[op.ticket_base + r * op.num_kv_heads + h], S)) {
    for (int idx = threadIdx.x; idx < rows * (D / 2); idx += PK_THREADS) {
      int rr = idx / (D / 2), d = (idx % (D / 2)) * 2;
      // online merge over the splits, 8 records in flight per round trip
      float M = -INFINITY, L = 0.f, O0 = 0.f, O1 = 0.f;
      for (int s0 = 0; s0 < S; s0 += 8) {
        float mv[8], lv[8], o0[8], o1[8];
#pragma unroll
        for (int u = 0; u < 8; u++) {
          if (s0 + u < S) {
            const float* rc = rec_base + (size_t)(s0 + u) * kAttnRecFloats + rr * (D + 2);
            mv[u] = ld_agent(rc + D);
            lv[u] = ld_agent(rc + D + 1);
            o0[u] = ld_agent(rc + d);
            o1[u] = ld_agent(rc + d + 1);
          } else {
            mv[u] = -INFINITY; lv[u] = 0.f; o0[u] = 0.f; o1[u] = 0.f;
          }
        }
        float mb = M;
#pragma unroll
        for (int u = 0; u < 8; u++) mb = fmaxf(mb, mv[u]);
        float f0 = M == -INFINITY ? 0.f : exp2f(M - mb);
        L *= f0; O0 *= f0; O1 *= f0;
#pragma unroll
        for (int u = 0; u < 8; u++) {
          float f = mv[u] == -INFINITY ? 0.f : exp2f(mv[u] - mb);
          L += lv[u] * f; O0 += o0[u] * f; O1 += o1[u] * f;
        }
        M = mb;
      }
      float inv = L > 0.f ? 1.f / L : 0.f;
      int j = rr / G, g = rr % G;
      st_agent_u32(op.out + (size_t)(t0 + j) * op.out_ld + (size_t)(h * G + g) * D + d,
                   pack2<DT_BF16>(O0 * inv, O1 * inv));
    }
  }
  signal_event(a, t);
}

// ------------------------------------------------------------ batch manager
// Offline-mode prepare_next_batch (persistent_kernel.cuh:169-322), run by one
// thread; integer logic identical to the CPU restatement in the oracle.
__device__ void task_prepare(const KernelArgs& a, const TaskDesc& t, int task_id, Shared& sm) {
  if (!wait_event(a, t, task_id, sm)) return;
  if (threadIdx.x == 0) {
    const BatchMeta& s = a.meta;
    const int MR = s.max_requests, MT = s.max_tokens, MP = s.max_pages, PS = s.page_size, MSL = s.max_seq_len;
    int head = *s.page_queue_head, tail = *s.page_queue_tail;
    for (int i = 0; i < MR; i++) {
      int rid = s.request_ids[i];
      if (rid == -1) continue;
      int step = s.step[rid], qo = s.qo_indptr[i], nt = s.qo_indptr[i + 1] - qo, plen = s.prompt_lengths[rid];
      for (int j = 0; j < nt; j++)
        if (step + j + 1 >= plen && step + j + 1 < MSL)
          s.tokens[(size_t)rid * MSL + step + j + 1] =
              (int64_t)__hip_atomic_load(reinterpret_cast<uint64_t*>(s.output_tokens + qo + j), __ATOMIC_RELAXED,
                                         __HIP_MEMORY_SCOPE_AGENT);
      s.step[rid] = step + nt;
      if ((step + nt + 1 >= MSL) ||
          ((s.tokens[(size_t)rid * MSL + step + nt] == s.eos_token_id) && (step + nt >= plen))) {
        s.request_ids[i] = -1;
        int kp = s.kv_indptr[i], npg = s.kv_indptr[i + 1] - kp;
        for (int j = 0; j < npg; j++) { s.page_queue[tail % MP] = s.kv_indices[kp + j]; tail++; }
      }
    }
    // the page-table snapshot lives in LDS (xs reused as int32)
    int* snap = reinterpret_cast<int*>(sm.xs);
    int all = s.kv_indptr[MR];
    for (int i = 0; i < all && i < XS_ELEMS / 2; i++) snap[i] = s.kv_indices[i];
    int nreq = 0, ntok = 0, npg = 0;
    for (int i = 0; i < MR; i++) {
      int rid = s.request_ids[i];
      if (rid == -1) continue;
      int kp = s.kv_indptr[i], nold = s.kv_indptr[i + 1] - kp;
      s.request_ids[nreq] = rid;
      s.qo_indptr[nreq] = ntok;
      s.kv_indptr[nreq] = npg;
      int step = s.step[rid];
      int nnew = s.prompt_lengths[rid] - step;
      nnew = nnew > 0 ? (nnew < MT - ntok ? nnew : MT - ntok) : (1 < MT - ntok ? 1 : MT - ntok);
      for (int j = 0; j < nnew; j++) s.input_tokens[ntok + j] = s.tokens[(size_t)rid * MSL + step + j];
      int nnp = (step + nnew + PS - 1) / PS;
      s.last_page_len[nreq] = (step + nnew) % PS;
      for (int j = 0; j < nold; j++) s.kv_indices[npg + j] = snap[kp + j];
      for (int j = nold; j < nnp; j++) { s.kv_indices[npg + j] = s.page_queue[head % MP]; head++; }
      npg += nnp;
      ntok += nnew;
      nreq++;
    }
    while (nreq < MR && ntok < MT) {
      int nid = *s.next_request_id;
      if (nid >= s.total_requests) break;
      s.request_ids[nreq] = nid;
      s.qo_indptr[nreq] = ntok;
      s.kv_indptr[nreq] = npg;
      int nnew = s.prompt_lengths[nid] < MT - ntok ? s.prompt_lengths[nid] : MT - ntok;
      for (int j = 0; j < nnew; j++) s.input_tokens[ntok + j] = s.tokens[(size_t)nid * MSL + j];
      int nnp = (nnew + PS - 1) / PS;
      s.last_page_len[nreq] = nnew % PS;
      for (int j = 0; j < nnp; j++) { s.kv_indices[npg + j] = s.page_queue[head % MP]; head++; }
      ntok += nnew;
      npg += nnp;
      nreq++;
      *s.next_request_id = nid + 1;
    }
    for (int i = nreq; i < MR; i++) s.request_ids[i] = -1;
    for (int i = nreq; i <= MR; i++) { s.qo_indptr[i] = ntok; s.kv_indptr[i] = npg; }
    *s.page_queue_head = head;
    *s.page_queue_tail = tail;
    s.status[1] = ntok != 0;
  }
  signal_event(a, t);
}

// ------------------------------------------------------------ kernel
__global__ __launch_bounds__(PK_THREADS, 1) void pk_worker_kernel(KernelArgs a) {
  __shared__ Shared sm;
  const int w = blockIdx.x;
  const int q0 = a.queue_offsets[w], q1 = a.queue_offsets[w + 1];
  // this worker's task descriptors move to LDS, 256 at a time
  auto load_descs = [&](int first) __attribute__((always_inline)) {
    const int n = q1 - first < 256 ? q1 - first : 256;
    const int words = (int)(sizeof(TaskDesc) / 4);
    for (int i = threadIdx.x; i < n * words; i += PK_THREADS) {
      int k = i / words, e = i % words;
      reinterpret_cast<uint32_t*>(&sm.tq[k])[e] = reinterpret_cast<const uint32_t*>(&a.tasks[a.queue[first + k]])[e];
    }
  };
  load_descs(q0);
  if (threadIdx.x == 0) {
    sm.flag = 1;
    sm.last_op = -1;
    sm.last_T = 0;
  }
  __syncthreads();
  for (int q = q0; q < q1; q++) {
    if (q > q0 && (q - q0) % 256 == 0) {
      __syncthreads();
      load_descs(q);
      __syncthreads();
    }
    const int tid = a.queue[q];
    const TaskDesc& t = sm.tq[(q - q0) % 256];
    const OpDesc& op = a.ops[t.op];
    if (a.profile && threadIdx.x == 0) {
      a.profile[(size_t)tid * 8] = now_10ns();
      a.profile[(size_t)tid * 8 + 3] = (uint64_t)w;
    }
    const int tm8 = op.max_tokens > 1;
    const bool gemv = op.type == TASK_LINEAR || op.type == TASK_RMSNORM_LINEAR ||
                      op.type == TASK_RMSNORM_LINEAR_SILU || op.type == TASK_RMSNORM_LINEAR_ARGMAX;
    if (!gemv && threadIdx.x == 0) sm.last_op = -1;  // attention / embed / batch tasks reuse xs
    switch (op.type) {
      case TASK_EMBED: task_embed(a, t, tid, sm); break;
      case TASK_LINEAR:
        if (tm8) task_gemv<8, EPI_LIN>(a, t, tid, sm); else task_gemv<1, EPI_LIN>(a, t, tid, sm);
        break;
      case TASK_RMSNORM_LINEAR:
        if (tm8) task_gemv<8, EPI_NORM>(a, t, tid, sm); else task_gemv<1, EPI_NORM>(a, t, tid, sm);
        break;
      case TASK_RMSNORM_LINEAR_SILU:
        if (tm8) task_gemv<8, EPI_SILU>(a, t, tid, sm); else task_gemv<1, EPI_SILU>(a, t, tid, sm);
        break;
      case TASK_RMSNORM_LINEAR_ARGMAX:
        if (tm8) task_gemv<8, EPI_ARGMAX>(a, t, tid, sm); else task_gemv<1, EPI_ARGMAX>(a, t, tid, sm);
        break;
      case TASK_ATTENTION: {
        const int r = t.i0;
        const int nt = a.meta.qo_indptr[r + 1] - a.meta.qo_indptr[r];
        if (nt * (op.num_q_heads / op.num_kv_heads) <= 4) task_attention<4>(a, t, tid, sm);
        else task_attention<16>(a, t, tid, sm);
        break;
      }
      case TASK_PREPARE_BATCH: task_prepare(a, t, tid, sm); break;
      default: break;
    }
    // GEMV tasks need no trailing barrier: the next task's first LDS access
    // comes after its own [X] barrier, which the sync wave reaches only after
    // publishing this task, so the compute waves run ahead and put the next
    // task's weights in flight meanwhile
    if (!gemv) __syncthreads();
    if (a.profile && threadIdx.x == 0) a.profile[(size_t)tid * 8 + 2] = now_10ns();
    if (!sm.flag) break;  // a dependency never arrived: leave the queue
  }
}

// Batch state initialisation (persistent_kernel.cuh:107-132).
__global__ void pk_init_batch_kernel(BatchMeta s) {
  if (threadIdx.x == 0 && blockIdx.x == 0) {
    for (int i = 0; i < s.total_requests; i++) s.step[i] = 0;
    *s.next_request_id = 0;
    for (int i = 0; i < s.max_requests; i++) s.request_ids[i] = -1;
    for (int i = 0; i < s.max_requests + 1; i++) { s.qo_indptr[i] = 0; s.kv_indptr[i] = 0; }
    *s.page_queue_head = 0;
    *s.page_queue_tail = s.max_pages;
    for (int i = 0; i < s.max_pages; i++) s.page_queue[i] = i;
  }
}

__global__ void pk_fill_u32_kernel(uint32_t* p, size_t n, uint32_t v) {
  for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (size_t)gridDim.x * blockDim.x) p[i] = v;
}

// ------------------------------------------------------------ host handle
struct Handle {
  int device = 0;
  int num_workers = 0;
  size_t n_ops = 0, n_tasks = 0, n_events = 0;
  OpDesc* d_ops = nullptr;
  TaskDesc* d_tasks = nullptr;
  int* d_qoff = nullptr;
  int* d_queue = nullptr;
  uint32_t* d_events = nullptr;
  uint32_t* d_tickets = nullptr;
  float* d_scratch = nullptr;
  int* d_status = nullptr;
  int* d_owned_meta = nullptr;  // request_ids, next_request_id, page_queue, head, tail
  BatchMeta meta;
  uint32_t epoch = 0;
  long long spin_limit = 1ll << 26;
  uint64_t* profile = nullptr;
};

}  // namespace pk
}  // namespace yr

using namespace yr;
using namespace yr::pk;

static int hip_ok(hipError_t e, const char* what) { return check_hip(e, what); }

extern "C" {

int yr_pk_create(const yr_pk_graph* gp, const yr_pk_meta* mp, yr_pk_handle** out) {
  const Graph* g = reinterpret_cast<const Graph*>(gp);
  if (!g || !mp || !out) return fail(YR_E_INVALID, "yr_pk_create: null argument");
  *out = nullptr;
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) return fail(YR_E_NODEVICE, "yr_pk_create: no HIP device");
  hipDeviceProp_t prop;
  if (hipGetDeviceProperties(&prop, dev) != hipSuccess) return fail(YR_E_NODEVICE, "yr_pk_create: device query");
  int occ = 0;
  if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&occ, reinterpret_cast<const void*>(pk_worker_kernel), PK_THREADS,
                                                   0) != hipSuccess)
    return fail(YR_E_HIP, "yr_pk_create: occupancy query failed");
  if (g->num_workers > occ * prop.multiProcessorCount)
    return fail(YR_E_INVALID, "yr_pk_create: %d workers cannot be co-resident (%d CUs x %d)", g->num_workers,
                prop.multiProcessorCount, occ);
  Handle* h = new Handle();
  h->device = dev;
  h->num_workers = g->num_workers;
  h->n_ops = g->ops.size();
  h->n_tasks = g->tasks.size();
  h->n_events = g->events.size();
  // queues flattened
  std::vector<int> qoff(g->num_workers + 1, 0), queue;
  for (int w = 0; w < g->num_workers; w++) {
    qoff[w] = (int)queue.size();
    queue.insert(queue.end(), g->queues[w].begin(), g->queues[w].end());
  }
  qoff[g->num_workers] = (int)queue.size();
  int rc = YR_OK;
#define YRA(ptr, bytes)                                                     \
  if (rc == YR_OK) rc = hip_ok(hipMalloc((void**)&(ptr), (bytes) ? (bytes) : 16), "hipMalloc")
  YRA(h->d_ops, sizeof(OpDesc) * h->n_ops);
  YRA(h->d_tasks, sizeof(TaskDesc) * h->n_tasks);
  YRA(h->d_qoff, sizeof(int) * qoff.size());
  YRA(h->d_queue, sizeof(int) * queue.size());
  YRA(h->d_events, sizeof(uint32_t) * h->n_events);
  YRA(h->d_tickets, sizeof(uint32_t) * (g->num_tickets + 1));
  YRA(h->d_scratch, sizeof(float) * (g->scratch_floats + 4));
  YRA(h->d_status, sizeof(int) * 4);
  const int MR = g->cfg.max_requests, MP = g->cfg.max_pages;
  YRA(h->d_owned_meta, sizeof(int) * (MR + 1 + MP + 2));
#undef YRA
  if (rc == YR_OK) rc = hip_ok(hipMemcpy(h->d_ops, g->ops.data(), sizeof(OpDesc) * h->n_ops, hipMemcpyHostToDevice), "copy ops");
  if (rc == YR_OK) rc = hip_ok(hipMemcpy(h->d_tasks, g->tasks.data(), sizeof(TaskDesc) * h->n_tasks, hipMemcpyHostToDevice), "copy tasks");
  if (rc == YR_OK) rc = hip_ok(hipMemcpy(h->d_qoff, qoff.data(), sizeof(int) * qoff.size(), hipMemcpyHostToDevice), "copy queues");
  if (rc == YR_OK && queue.size()) rc = hip_ok(hipMemcpy(h->d_queue, queue.data(), sizeof(int) * queue.size(), hipMemcpyHostToDevice), "copy queues");
  if (rc == YR_OK) rc = hip_ok(hipMemset(h->d_events, 0, sizeof(uint32_t) * h->n_events), "clear events");
  if (rc == YR_OK) rc = hip_ok(hipMemset(h->d_tickets, 0, sizeof(uint32_t) * (g->num_tickets + 1)), "clear tickets");
  if (rc == YR_OK) rc = hip_ok(hipMemset(h->d_status, 0, sizeof(int) * 4), "clear status");
  if (rc != YR_OK) {
    yr_pk_destroy(reinterpret_cast<yr_pk_handle*>(h));
    return rc;
  }
  BatchMeta& m = h->meta;
  m.step = mp->step;
  m.tokens = mp->tokens;
  m.input_tokens = mp->input_tokens;
  m.output_tokens = mp->output_tokens;
  m.num_new_tokens = mp->num_new_tokens;
  m.prompt_lengths = mp->prompt_lengths;
  m.qo_indptr = mp->qo_indptr;
  m.kv_indptr = mp->paged_kv_indptr;
  m.kv_indices = mp->paged_kv_indices;
  m.last_page_len = mp->paged_kv_last_page_len;
  m.request_ids = h->d_owned_meta;
  m.next_request_id = h->d_owned_meta + MR;
  m.page_queue = h->d_owned_meta + MR + 1;
  m.page_queue_head = h->d_owned_meta + MR + 1 + MP;
  m.page_queue_tail = h->d_owned_meta + MR + 2 + MP;
  m.status = h->d_status;
  m.max_requests = MR;
  m.max_tokens = g->cfg.max_tokens;
  m.max_pages = MP;
  m.page_size = g->cfg.page_size;
  m.max_seq_len = g->cfg.max_seq_len;
  m.total_requests = g->cfg.total_requests;
  m.eos_token_id = g->cfg.eos_token_id;
  if (!m.qo_indptr || !m.kv_indptr || !m.kv_indices || !m.last_page_len) {
    yr_pk_destroy(reinterpret_cast<yr_pk_handle*>(h));
    return fail(YR_E_INVALID, "yr_pk_create: qo_indptr / paged_kv_* meta tensors are required");
  }
  *out = reinterpret_cast<yr_pk_handle*>(h);
  return YR_OK;
}

int yr_pk_init_batch(yr_pk_handle* hp, void* stream) {
  Handle* h = reinterpret_cast<Handle*>(hp);
  if (!h) return fail(YR_E_INVALID, "yr_pk_init_batch: null handle");
  if (!h->meta.step || !h->meta.tokens || !h->meta.prompt_lengths || !h->meta.input_tokens || !h->meta.output_tokens)
    return fail(YR_E_INVALID, "yr_pk_init_batch: step/tokens/prompt_lengths/input_tokens/output_tokens are required");
  hipLaunchKernelGGL(pk_init_batch_kernel, dim3(1), dim3(64), 0, (hipStream_t)stream, h->meta);
  YR_CHECK_LAUNCH("pk_init_batch_kernel");
  return YR_OK;
}

int yr_pk_launch(yr_pk_handle* hp, void* stream) {
  Handle* h = reinterpret_cast<Handle*>(hp);
  if (!h) return fail(YR_E_INVALID, "yr_pk_launch: null handle");
  hipStream_t st = (hipStream_t)stream;
  // counters are monotonic; re-base them well before 32-bit wrap
  if (h->epoch >= (1u << 20)) {
    hipLaunchKernelGGL(pk_fill_u32_kernel, dim3(64), dim3(256), 0, st, h->d_events, h->n_events, 0u);
    YR_CHECK_LAUNCH("pk_fill_u32_kernel");
    h->epoch = 0;
  }
  h->epoch++;
  KernelArgs a;
  a.ops = h->d_ops;
  a.tasks = h->d_tasks;
  a.queue_offsets = h->d_qoff;
  a.queue = h->d_queue;
  a.events = h->d_events;
  a.tickets = h->d_tickets;
  a.scratch = h->d_scratch;
  a.meta = h->meta;
  a.epoch = h->epoch;
  a.num_workers = h->num_workers;
  a.spin_limit = h->spin_limit;
  a.profile = h->profile;
  void* args[] = {&a};
  hipError_t e = hipLaunchCooperativeKernel(reinterpret_cast<const void*>(pk_worker_kernel), dim3(h->num_workers),
                                            dim3(PK_THREADS), args, 0, st);
  if (e != hipSuccess) return check_hip(e, "hipLaunchCooperativeKernel(pk_worker_kernel)");
  return YR_OK;
}

int yr_pk_set_spin_limit(yr_pk_handle* hp, long long polls) {
  Handle* h = reinterpret_cast<Handle*>(hp);
  if (!h || polls <= 0) return fail(YR_E_INVALID, "yr_pk_set_spin_limit: bad arguments");
  h->spin_limit = polls;
  return YR_OK;
}

int yr_pk_set_profiler(yr_pk_handle* hp, uint64_t* buffer, size_t entries) {
  Handle* h = reinterpret_cast<Handle*>(hp);
  if (!h) return fail(YR_E_INVALID, "yr_pk_set_profiler: null handle");
  if (buffer && entries < h->n_tasks * 8)
    return fail(YR_E_INVALID, "yr_pk_set_profiler: buffer needs %zu entries", h->n_tasks * 8);
  h->profile = buffer;
  return YR_OK;
}

int yr_pk_status(yr_pk_handle* hp, int* status4) {
  Handle* h = reinterpret_cast<Handle*>(hp);
  if (!h || !status4) return fail(YR_E_INVALID, "yr_pk_status: bad arguments");
  hipError_t e = hipMemcpy(status4, h->d_status, sizeof(int) * 4, hipMemcpyDeviceToHost);
  if (e != hipSuccess) return check_hip(e, "yr_pk_status");
  if (status4[0]) return fail(YR_E_TIMEOUT, "persistent kernel watchdog fired waiting in task %d", status4[2]);
  if (status4[3])
    return fail(YR_E_INVALID, "attention task %d: more than 16 query rows per kv head or 512 positions per split",
                status4[3] - 1);
  return YR_OK;
}

int yr_pk_reset_status(yr_pk_handle* hp) {
  Handle* h = reinterpret_cast<Handle*>(hp);
  if (!h) return fail(YR_E_INVALID, "yr_pk_reset_status: null handle");
  // clear the flags and re-base the counters (a watchdog exit leaves them short)
  if (hipMemset(h->d_status, 0, sizeof(int) * 4) != hipSuccess) return fail(YR_E_HIP, "reset status");
  if (hipMemset(h->d_events, 0, sizeof(uint32_t) * h->n_events) != hipSuccess) return fail(YR_E_HIP, "reset events");
  h->epoch = 0;
  return YR_OK;
}

void yr_pk_destroy(yr_pk_handle* hp) {
  Handle* h = reinterpret_cast<Handle*>(hp);
  if (!h) return;
  void* ptrs[] = {h->d_ops, h->d_tasks, h->d_qoff, h->d_queue, h->d_events, h->d_tickets, h->d_scratch, h->d_status,
                  h->d_owned_meta};
  for (void* p : ptrs)
    if (p) (void)hipFree(p);
  delete h;
}

}  // extern "C"
