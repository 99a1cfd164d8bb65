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
constexpr int OUT_ELEMS = 16384;  // GEMV partial-sum slots (32 KiB as float)

// An attention task's request geometry and the page ids of its first
// blocks, read from the batch metadata when the worker loads its task
// descriptors: the metadata is written by the host or by the previous
// launch's prepare_batch task and does not change before this launch's last
// attention task, so the task itself starts its K/V and q loads without a
// dependent metadata round trip.
struct AttnPre {
  int t0, nt, pb, np, base, c0, c1, ok;
  int id[14];     // pages (A, B) of block w, for compute waves w < 7
  int pg_tok[4];  // pages of new tokens 0..3
  int pad[6];
};
constexpr int kPreMax = 64;
constexpr uint8_t kPreNone = 255;

struct Shared {
  uint16_t xs[XS_ELEMS];          // activations (bf16), [token][KB]
  uint16_t outs[OUT_ELEMS];       // GEMV partial-sum slots (float)
  float red[PK_WAVES * 16 * 2];   // small reductions
  float attn_p[PK_WAVES][16][64]; // attention probabilities per wave
  float attn_ml[PK_WAVES][16][2];
  TaskDesc tq[256];               // this worker's first 256 task descriptors
  int tq_id[256];                 // their task ids
  AttnPre pre[kPreMax];           // attention geometry / page ids, read when descriptors load
  uint8_t pre_of[256];            // descriptor slot -> pre entry (kPreNone: none)
  int pre_n;
  int flag;                       // last wait succeeded (0 after a watchdog exit)
  int last_op;                    // op whose activations are staged in xs (-1: none)
  int last_T;
  int norm_rows;                  // batch > 1: rows staged raw, normalized by waves 0..T-1
  int coop_stage;                 // batch > 1: block 0 of the input is staged by all waves after [X]
  KernelArgs args;                // this launch's arguments, for the task functions
};

// One workgroup per CU: the worker's LDS, addressed directly by the task
// functions (which are separate functions, so that each task type gets its
// own register allocation, and read their arguments from here instead of
// through generic pointers).
__shared__ Shared g_sm;

// The op table is read-only for a whole launch: reading it through the
// constant address space lets uniform field loads become scalar loads, which
// never queue behind (or wait for) the vector memory traffic of a task.
using OpRef = const __attribute__((address_space(4))) OpDesc&;
__device__ __forceinline__ OpRef op_of(const KernelArgs& a, int i) {
  return reinterpret_cast<const __attribute__((address_space(4))) OpDesc*>(
      reinterpret_cast<uintptr_t>(a.ops))[i];
}

// Thread index behind an empty volatile asm: values derived from it are
// recomputed inside each task instead of being hoisted out of the worker loop
// (hoisted lane addresses stay live across every task and push the kernel
// into scratch spills, and a spill reload is a full memory round trip).
__device__ __forceinline__ int tix() {
  int t = (int)threadIdx.x;
  asm volatile("" : "+v"(t));
  return t;
}

// Workgroup barrier for LDS hand-offs only.  __syncthreads() carries a
// workgroup release fence, which waits for every outstanding global store of
// the wave (a memory round trip after link / cache / record stores); here the
// wave only waits for its own LDS operations.
__device__ __forceinline__ void lds_sync() {
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0)
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
}

#ifndef YR_PK_EVENT_SLEEP
#define YR_PK_EVENT_SLEEP 16  // s_sleep between event-counter polls of a whole-workgroup wait (x 64 clocks)
#endif
#ifndef YR_PK_LINK_SLEEP
#define YR_PK_LINK_SLEEP 2  // s_sleep between re-reads of stale link words (x 64 clocks)
#endif
#ifndef YR_PK_LINK_NB
#define YR_PK_LINK_NB 24    // link-word loads per lane in flight when staging a batch-1 input
#endif
// ------------------------------------------------------------ protocol
__device__ __forceinline__ bool aborted(const KernelArgs& a) {
  return __hip_atomic_load(gptr(a.meta.status), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) != 0;
}

// Whole-workgroup wait until events[e] >= wait_count * epoch.  Returns false
// when the watchdog fired here or elsewhere.
__device__ __forceinline__ uint64_t now_10ns() { return __builtin_amdgcn_s_memrealtime(); }

constexpr int POLL_T = (PK_WAVES - 1) * kWave;  // first lane of the sync wave (no weight loads)

__device__ bool wait_event(const KernelArgs& a, const TaskDesc& t, int task_id, Shared& sm) {
  if (t.wait_event < 0) {
    if (a.profile && tix() == POLL_T) gptr(a.profile)[(size_t)task_id * 8 + 1] = now_10ns();
    return true;
  }
  if (tix() == POLL_T) {
    const uint32_t need = (uint32_t)t.wait_count * a.epoch;
    long long spins = 0;
    int ok = 1;
    for (;;) {
      uint32_t v = __hip_atomic_load(gptr(&a.events[t.wait_event]), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      if ((int32_t)(v - need) >= 0) break;
      if ((spins & 255) == 255 && aborted(a)) { ok = 0; break; }
      if (++spins > a.spin_limit) {
        __hip_atomic_store(gptr(a.meta.status + 2), task_id, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        __hip_atomic_store(gptr(a.meta.status), 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        ok = 0;
        break;
      }
      __builtin_amdgcn_s_sleep(YR_PK_EVENT_SLEEP);
    }
    if (a.profile) gptr(a.profile)[(size_t)task_id * 8 + 1] = now_10ns();
    sm.flag = ok;
  }
  __syncthreads();
  return sm.flag != 0;
}

// Publish completion: every thread's stores are complete, then one arrival.
// Outputs that are link tensors need not be complete: their readers check
// tags, so only the other stores of the task are waited for.
__device__ void signal_event(const KernelArgs& a, const TaskDesc& t, bool link_out = false) {
  if (!link_out) wait_vm();  // every wave's stores complete before the one signal
  lds_sync();
  if (tix() == POLL_T && t.trigger_event >= 0)
    __hip_atomic_fetch_add(gptr(&a.events[t.trigger_event]), 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

__device__ __forceinline__ uint32_t ld_agent_u32(const void* p) {
  return __hip_atomic_load(gptr(reinterpret_cast<const uint32_t*>(p)), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void st_agent_u32(void* p, uint32_t v) {
  __hip_atomic_store(gptr(reinterpret_cast<uint32_t*>(p)), v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ uint4 ld_agent_u128(const void* p) {
  const uint64_t* q = reinterpret_cast<const uint64_t*>(p);
  uint64_t lo = __hip_atomic_load(gptr(q), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  uint64_t hi = __hip_atomic_load(gptr(q + 1), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  return make_uint4((uint32_t)lo, (uint32_t)(lo >> 32), (uint32_t)hi, (uint32_t)(hi >> 32));
}
__device__ __forceinline__ void st_agent_u128(void* p, uint4 v) {
  uint64_t* q = reinterpret_cast<uint64_t*>(p);
  __hip_atomic_store(gptr(q), (uint64_t)v.x | ((uint64_t)v.y << 32), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  __hip_atomic_store(gptr(q + 1), (uint64_t)v.z | ((uint64_t)v.w << 32), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}


// ------------------------------------------------------------ link tensors
__device__ __forceinline__ uint32_t link_tag(const KernelArgs& a, int op) {
  return (a.epoch << kLinkOpBits) | (uint32_t)op;
}
// store the bf16 pair `pair` at (even) element `e` of a link tensor
__device__ __forceinline__ void link_store(uint16_t* base, size_t e, uint32_t pair, uint32_t tag) {
  __hip_atomic_store(gptr(reinterpret_cast<uint64_t*>(base) + e / 2), (uint64_t)pair | ((uint64_t)tag << 32),
                     __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
// A word that still carries another tag is re-read until it matches; the
// spin shares the watchdog of event waits.  Returns false after a timeout /
// abort (the caller's data is then garbage, and the status flag is set).
__device__ __forceinline__ bool link_spin(const KernelArgs& a, const uint64_t* w, uint32_t tag, uint64_t& v) {
  long long spins = 0;
  for (;;) {
    v = __hip_atomic_load(gptr(w), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    if ((uint32_t)(v >> 32) == tag) return true;
    if ((spins & 255) == 255 && aborted(a)) return false;
    if (++spins > a.spin_limit) {
      __hip_atomic_store(gptr(a.meta.status + 2), -1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      __hip_atomic_store(gptr(a.meta.status), 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      return false;
    }
    __builtin_amdgcn_s_sleep(YR_PK_LINK_SLEEP);
  }
}
// the bf16 pair at (even) element e, waiting for this launch's producer
__device__ __forceinline__ uint32_t link_load(const KernelArgs& a, const uint16_t* base, size_t e, uint32_t tag) {
  const uint64_t* w = reinterpret_cast<const uint64_t*>(base) + e / 2;
  uint64_t v = __hip_atomic_load(gptr(w), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  if ((uint32_t)(v >> 32) != tag) link_spin(a, w, tag, v);
  return (uint32_t)v;
}
// Eight elements (e % 8 == 0) of a link tensor as two 16-byte loads; issue
// several with link8_issue before completing any with link8_take.
struct Link8 {
  uint4 w0, w1;  // words (pair, tag) x 2 each
};
__device__ __forceinline__ Link8 link8_issue(const uint16_t* base, size_t e) {
  const uint16_t* p = base + 2 * e;  // 4 bytes per element
  Link8 r;
  r.w0 = ld_agent_u128(p);
  r.w1 = ld_agent_u128(p + 8);
  return r;
}
__device__ __forceinline__ bool link8_ok(const Link8& r, uint32_t tag) {
  return r.w0.y == tag && r.w0.w == tag && r.w1.y == tag && r.w1.w == tag;
}
__device__ __forceinline__ uint4 link8_data(const Link8& r) { return make_uint4(r.w0.x, r.w0.z, r.w1.x, r.w1.z); }
// One step of a wave-level retry loop over stale link words: false once the
// watchdog fired or the launch was aborted (status flag set).
__device__ __forceinline__ bool link_retry(const KernelArgs& a, long long& spins) {
  if ((spins & 255) == 255 && aborted(a)) return false;
  if (++spins > a.spin_limit) {
    __hip_atomic_store(gptr(a.meta.status + 2), -1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    __hip_atomic_store(gptr(a.meta.status), 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    return false;
  }
  __builtin_amdgcn_s_sleep(YR_PK_LINK_SLEEP);
  return true;
}
// eight elements of either kind of tensor (plain: one agent-coherent load)
__device__ __forceinline__ Link8 act8_issue(bool link, const uint16_t* base, size_t e) {
  if (link) return link8_issue(base, e);
  Link8 r;
  r.w0 = ld_agent_u128(base + e);
  r.w1 = make_uint4(0, 0, 0, 0);
  return r;
}
__device__ __forceinline__ bool act8_ok(bool link, const Link8& r, uint32_t tag) { return !link || link8_ok(r, tag); }
__device__ __forceinline__ uint4 act8_data(bool link, const Link8& r) { return link ? link8_data(r) : r.w0; }

__device__ __forceinline__ int active_tokens(const KernelArgs& a, OpRef op) {
  int n = (int)ld_agent_u32(a.meta.qo_indptr + a.meta.max_requests);
  return n < op.max_tokens ? n : op.max_tokens;
}

// ------------------------------------------------------------ embedding
__device__ __forceinline__ void task_embed(const KernelArgs& a, const TaskDesc& t, int task_id, Shared& sm) {
  OpRef op = op_of(a, t.op);
  if (!wait_event(a, t, task_id, sm)) return;
  const int T = active_tokens(a, op);
  for (int b = 0; b < T; b++) {
    uint64_t tok = (uint64_t)__hip_atomic_load(gptr(reinterpret_cast<const uint64_t*>(op.tokens_in + b)), __ATOMIC_RELAXED,
                                               __HIP_MEMORY_SCOPE_AGENT);
    if (tok >= (uint64_t)op.vocab) tok = 0;  // out-of-range ids read row 0
    const uint16_t* src = op.table + tok * (uint64_t)op.K + t.row0;
    if (op.flags & OPF_OUT_LL) {
      const uint32_t tag = link_tag(a, t.op);
      const size_t e0 = (size_t)b * op.out_ld + t.row0;
      for (int i = tix() * 8; i < t.rows; i += PK_THREADS * 8) {
        const uint4 v = ldg16(src + i);
        link_store(op.out, e0 + i, v.x, tag);
        link_store(op.out, e0 + i + 2, v.y, tag);
        link_store(op.out, e0 + i + 4, v.z, tag);
        link_store(op.out, e0 + i + 6, v.w, tag);
      }
    } else {
      uint16_t* dst = op.out + (size_t)b * op.out_ld + t.row0;
      for (int i = tix() * 8; i < t.rows; i += PK_THREADS * 8) st_agent_u128(dst + i, ldg16(src + i));
    }
  }
  signal_event(a, t, (op.flags & OPF_OUT_LL) != 0);
}

// Geometry of attention task (request r, split s): new tokens [t0, t0+nt),
// pages [pb, pb+np) of the page table, cached positions [0, base), of which
// this split reads [c0, c1).  With OPF_EMPTY_MERGER the cached positions go
// to splits 0 .. S-2 and the last split -- which appends the new tokens,
// attends to them and merges the others' records -- reads none, so it is
// ready to merge as soon as the others' records arrive.
constexpr int kPage = 64;  // KV page size in positions (the builder accepts only this)

struct AttnGeom {
  int t0, nt, pb, np, base, c0, c1;
};

__device__ __forceinline__ AttnGeom attn_geom(const BatchMeta& m, OpRef op, int r, int s) {
  AttnGeom g;
  const int S = op.splits;
  g.t0 = gptr(m.qo_indptr)[r];
  g.nt = gptr(m.qo_indptr)[r + 1] - g.t0;
  g.pb = gptr(m.kv_indptr)[r];
  g.np = gptr(m.kv_indptr)[r + 1] - g.pb;
  const int lpl = gptr(m.last_page_len)[r];
  const int seq = g.nt > 0 ? (g.np - 1) * kPage + (lpl == 0 ? kPage : lpl) : 0;
  g.base = seq - g.nt;
  const int SC = S > 1 && (op.flags & OPF_EMPTY_MERGER) ? S - 1 : S;  // splits that read cached positions
  int chunk = (g.base + SC - 1) / SC;
  chunk = (chunk + 15) & ~15;
  g.c0 = s * chunk < g.base ? s * chunk : g.base;
  g.c1 = (s + 1) * chunk < g.base ? (s + 1) * chunk : g.base;
  return g;
}

// ------------------------------------------------------------ GEMV family
// Workgroup roles: waves 0..CW-1 stream weights and do the dot products; the
// sync wave (wave CW) never loads weights, so its dependency polls and
// activation loads never wait (vmcnt is in order) behind weight traffic.
//   compute waves: RING weight loads in flight -> [X] -> stream the unit range
//                  (consume one 1 KiB unit, issue the next) -> [O]
//   sync wave:     poll the event -> stage activations (+RMSNorm) -> [X]
//                  -> [O] -> epilogue, stores, publish
// Work is cut into units of 512 elements of one weight row (one 16-byte load
// per lane).  The RT x NC units of a staged block are split into CW equal
// contiguous row-major ranges, one per compute wave, so every wave streams the
// same number of bytes whatever the row count.  A wave keeps fp32 partial sums
// for its current row and adds them into LDS slot (row + wave) when the row
// (or its range) ends; (row, wave) pairs of one split never collide on a slot,
// and the epilogue adds a row's slots in wave order, so results do not depend
// on timing.  The code is kept loop-shaped and small on purpose: every task
// type runs its straight-line code once per task, and on gfx950 fetching
// instructions that fell out of the instruction cache costs more than the
// arithmetic it saves to unroll them.
enum { EPI_LIN = 0, EPI_NORM = 1, EPI_SILU = 2, EPI_ARGMAX = 3 };
constexpr int CW = PK_WAVES - 1;           // compute waves
constexpr int SYNC_T0 = CW * kWave;        // first thread of the sync wave
#ifndef YR_PK_RING
#define YR_PK_RING 12
#endif
#ifndef YR_PK_RING8
#define YR_PK_RING8 16  // batch 2..8 (packed; 12 / 16: 5.251 / 5.136 ms, 16 tokens 6.95 / 7.16 ms at 16)
#endif
#ifndef YR_PK_RING1
#define YR_PK_RING1 14  // batch 1 (sweep 10 / 12 / 14 / 16: 3.629 / 3.636 / 3.611 / 3.632 ms)
#endif
constexpr int RING = YR_PK_RING;           // weight loads in flight per compute lane (RING * 7 KiB per CU)
constexpr int kCpolSC1 = 16;               // buffer cache policy: agent-coherent (sc1)

// 128-bit agent-coherent loads of activations written by other CUs.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t rsrc_of(const void* p) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(p), 0, 0x7fffffff, 0x00020000);
}
__device__ __forceinline__ uint4 ld_sc1(__amdgpu_buffer_rsrc_t r, uint32_t byte_off) {
  return __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(r, byte_off, 0, kCpolSC1));
}

__device__ __forceinline__ f32x4 mfma_bf16(uint4 a, uint4 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8v, a), __builtin_bit_cast(bf16x8v, b), c,
                                                 0, 0, 0);
}

// Column e of staged activation row b (b < 8): 16-byte chunk e / 8 XOR b.
__device__ __forceinline__ int xs_swz(int b, int e) { return (((e >> 3) ^ b) << 3) | (e & 7); }

// Sync wave: rows [0, TM) of elements [k0, k0 + KB) of op.x into xs[b][KB];
// rows b >= T are zero.  16 loads per lane in flight.
// NRM (16-token batches, where K no longer fits one staged block): each
// value is normalized on the way in, x * (r_b * gamma) rounded to bf16, with
// the row factors r_b = rsqrt(mean(x_b^2) + eps) from row_rms_coop (in attn_ml).
template <int TM, bool NRM = false>
__device__ __forceinline__ void stage_x(OpRef op, int T, int KB, int k0, Shared& sm, int lane, int xoff = 0) {
  // groups of 64 chunks (one 16-byte load per lane): group m is row m / k,
  // chunks (m % k) * 64 + lane.  Row and group offsets are wave-uniform, so
  // a load is one buffer load at (lane * 16 + scalar offset), and groups past
  // the end load from beyond the buffer (zero, no memory access) into a junk
  // LDS line: the unrolled batch has no branches.
  const int k = KB >> 9, total = TM * k;
  const int nrec = __builtin_amdgcn_readfirstlane((int)((size_t)T * op.x_ld * 2));  // rows >= T read as zero
  const __amdgpu_buffer_rsrc_t r =
      __builtin_amdgcn_make_buffer_rsrc(const_cast<uint16_t*>(op.x), 0, nrec, 0x00020000);
  const uint32_t vo = lane * 16;
  const int row_bytes = op.x_ld * 2;
  uint16_t* const junk = reinterpret_cast<uint16_t*>(sm.red);
  constexpr int NB = TM == 1 ? 16 : 32;  // loads per lane in flight
  // NRM: this lane's gamma chunks of the block (k <= 4: KB <= XS_ELEMS / 16),
  // loaded once up front -- a gamma load per staged chunk would cost one
  // round trip through the CU's memory queue each
  uint4 gam[4];
  if constexpr (NRM) {
#pragma unroll
    for (int j = 0; j < 4; j++) gam[j] = j < k ? ldg16(op.norm + k0 + j * 512 + lane * 8) : make_uint4(0, 0, 0, 0);
  }
  for (int g = 0; g < total; g += NB) {
    const int mb0 = g / k, mc0 = g - mb0 * k;
    uint4 v[NB];
    int rb = mb0 * row_bytes + k0 * 2, co = mc0 * 1024;
#pragma unroll
    for (int u = 0; u < NB; u++) {
      const int off = g + u < total ? rb + co : 0x7ffffff0;
      v[u] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(r, vo, off, kCpolSC1));
      co += 1024;
      if (co == k * 1024) { co = 0; rb += row_bytes; }
    }
    // element (row b, column e) lives at b * KB + xs_swz(b, e): 16-byte
    // chunks XOR-permuted by row so that the MFMA B reads of 8 rows hit 8
    // different bank groups (identity for row 0, the batch-1 layout)
    int xr = mb0, xc = mc0;
#pragma unroll
    for (int u = 0; u < NB; u++) {
      uint16_t* dst = g + u < total ? sm.xs + xoff + xr * KB + xs_swz(xr, xc * 512 + lane * 8) : junk + lane * 8;
      if constexpr (NRM) {
        const float rb = sm.attn_ml[0][xr & 15][0];
        const uint4 gq = xc == 0 ? gam[0] : xc == 1 ? gam[1] : xc == 2 ? gam[2] : gam[3];
        const uint32_t xv[4] = {v[u].x, v[u].y, v[u].z, v[u].w}, gv[4] = {gq.x, gq.y, gq.z, gq.w};
        uint32_t o[4];
#pragma unroll
        for (int e = 0; e < 4; e++)
          o[e] = pack2<DT_BF16>(lo16<DT_BF16>(xv[e]) * (rb * lo16<DT_BF16>(gv[e])),
                                hi16<DT_BF16>(xv[e]) * (rb * hi16<DT_BF16>(gv[e])));
        v[u] = make_uint4(o[0], o[1], o[2], o[3]);
      }
      *reinterpret_cast<uint4*>(dst) = v[u];
      if (++xc == k) { xc = 0; xr++; }
    }
  }
}

// Block 0 of a batch > 1 input staged by all 8 waves at once (group g of
// stage_x goes to wave g % 8): every load is issued in one batch, so the
// rows cost one trip through the CU's memory queue (which holds the compute
// waves' weight prefetch) instead of one per batch of the sync wave.
template <int TM>
__device__ __forceinline__ void stage_x_coop(OpRef op, int T, int KB, Shared& sm, int wave, int lane) {
  const int k = KB >> 9, total = TM * k;  // <= 64 groups (KB <= XS_ELEMS / TM)
  const int nrec = __builtin_amdgcn_readfirstlane((int)((size_t)T * op.x_ld * 2));
  const __amdgpu_buffer_rsrc_t r =
      __builtin_amdgcn_make_buffer_rsrc(const_cast<uint16_t*>(op.x), 0, nrec, 0x00020000);
  const uint32_t vo = lane * 16;
  const int row_bytes = op.x_ld * 2;
  uint16_t* const junk = reinterpret_cast<uint16_t*>(sm.red);
  constexpr int NB = 8;
  uint4 v[NB];
#pragma unroll
  for (int u = 0; u < NB; u++) {
    const int g = wave + PK_WAVES * u;
    const int mb = g / k, mc = g - mb * k;
    const int off = g < total ? mb * row_bytes + mc * 1024 : 0x7ffffff0;
    v[u] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(r, vo, off, kCpolSC1));
  }
#pragma unroll
  for (int u = 0; u < NB; u++) {
    const int g = wave + PK_WAVES * u;
    const int mb = g / k, mc = g - mb * k;
    uint16_t* dst = g < total ? sm.xs + mb * KB + xs_swz(mb, mc * 512 + lane * 8) : junk + lane * 8;
    *reinterpret_cast<uint4*>(dst) = v[u];
  }
}

// 16-token batches, all 8 waves after [X]: r_b = rsqrt(mean(x_b^2) + eps)
// of every row (wave w takes rows w, w + 8), all of a wave's loads of a
// 2048-column stretch in flight at once, into attn_ml[0][b][0]; rows past T
// read as zero.  (The sync wave alone needed one trip through the CU's
// memory queue, behind the weight prefetch, per 2048 columns and 4 rows.)
template <int TM>
__device__ __forceinline__ void row_rms_coop(OpRef op, int T, Shared& sm, int wave, int lane) {
  const int K = op.K;
  const int nrec = __builtin_amdgcn_readfirstlane((int)((size_t)T * op.x_ld * 2));
  const __amdgpu_buffer_rsrc_t r =
      __builtin_amdgcn_make_buffer_rsrc(const_cast<uint16_t*>(op.x), 0, nrec, 0x00020000);
  const int row_bytes = op.x_ld * 2;
  constexpr int RPW = TM / PK_WAVES;  // rows per wave (2)
  float ss[RPW];
#pragma unroll
  for (int i = 0; i < RPW; i++) ss[i] = 0.f;
  for (int c = 0; c < K; c += 8 * kWave * 4) {
    uint4 v[RPW][4];
#pragma unroll
    for (int i = 0; i < RPW; i++)
#pragma unroll
      for (int u = 0; u < 4; u++) {
        const int col = c + (u * kWave + lane) * 8;
        const uint32_t vo = col < K ? (uint32_t)(lane * 16) : 0x7ffffff0u;
        v[i][u] = __builtin_bit_cast(
            uint4, __builtin_amdgcn_raw_buffer_load_b128(r, vo, (wave + PK_WAVES * i) * row_bytes + (c + u * kWave * 8) * 2,
                                                         kCpolSC1));
      }
#pragma unroll
    for (int i = 0; i < RPW; i++)
#pragma unroll
      for (int u = 0; u < 4; u++) {
        const uint32_t w4[4] = {v[i][u].x, v[i][u].y, v[i][u].z, v[i][u].w};
#pragma unroll
        for (int e = 0; e < 4; e++) {
          const float lo = lo16<DT_BF16>(w4[e]), hi = hi16<DT_BF16>(w4[e]);
          ss[i] += lo * lo + hi * hi;
        }
      }
  }
#pragma unroll
  for (int i = 0; i < RPW; i++) {
    const float t = wave_sum(ss[i]);
    if (lane == 0) sm.attn_ml[0][wave + PK_WAVES * i][0] = rsqrtf(t / (float)K + op.eps);
  }
}

// 16-token batches, all 8 waves after the row factors: block 0 of the input
// staged normalized, x * (r_b * gamma) rounded to bf16 (the values stage_x<16,
// true> writes), 512-column groups to waves by g % 8, one batch of loads.
template <int TM>
__device__ __forceinline__ void stage_x_coop_nrm(OpRef op, int T, int KB, Shared& sm, int wave, int lane) {
  const int k = KB >> 9, total = TM * k;  // <= 64 groups
  const int nrec = __builtin_amdgcn_readfirstlane((int)((size_t)T * op.x_ld * 2));
  const __amdgpu_buffer_rsrc_t r =
      __builtin_amdgcn_make_buffer_rsrc(const_cast<uint16_t*>(op.x), 0, nrec, 0x00020000);
  const uint32_t vo = lane * 16;
  const int row_bytes = op.x_ld * 2;
  constexpr int NB = 8;
  uint4 v[NB], gq[NB];
#pragma unroll
  for (int u = 0; u < NB; u++) {
    const int g = wave + PK_WAVES * u;
    const int mb = g / k, mc = g - mb * k;
    const int off = g < total ? mb * row_bytes + mc * 1024 : 0x7ffffff0;
    v[u] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(r, vo, off, kCpolSC1));
    gq[u] = g < total ? ldg16(op.norm + mc * 512 + lane * 8) : make_uint4(0, 0, 0, 0);
  }
#pragma unroll
  for (int u = 0; u < NB; u++) {
    const int g = wave + PK_WAVES * u;
    if (g < total) {
      const int mb = g / k, mc = g - mb * k;
      const float rb = sm.attn_ml[0][mb & 15][0];
      const uint32_t xv[4] = {v[u].x, v[u].y, v[u].z, v[u].w}, gv[4] = {gq[u].x, gq[u].y, gq[u].z, gq[u].w};
      uint32_t o[4];
#pragma unroll
      for (int e = 0; e < 4; e++)
        o[e] = pack2<DT_BF16>(lo16<DT_BF16>(xv[e]) * (rb * lo16<DT_BF16>(gv[e])),
                              hi16<DT_BF16>(xv[e]) * (rb * hi16<DT_BF16>(gv[e])));
      *reinterpret_cast<uint4*>(sm.xs + mb * KB + xs_swz(mb, mc * 512 + lane * 8)) = make_uint4(o[0], o[1], o[2], o[3]);
    }
  }
}


// Sync wave, link-tensor input (batch-1 graphs only): elements [k0, k0 + KB)
// of row 0 of op.x into xs[0][KB].  A lane loads chunks of four elements (one
// 16-byte buffer load = two tagged words, each single-copy atomic), 24 chunks
// in flight; a batch is re-read until every word carries the tag of this
// launch's producing op.
__device__ __forceinline__ void stage_x_link(const KernelArgs& a, OpRef op, int KB, int k0, Shared& sm, int lane) {
  const uint32_t tag = link_tag(a, op.x_src);
  const int total = KB >> 2;
  const __amdgpu_buffer_rsrc_t r =
      __builtin_amdgcn_make_buffer_rsrc(const_cast<uint16_t*>(op.x) + 2 * k0, 0, total * 16, 0x00020000);
  constexpr int NB = YR_PK_LINK_NB;
  for (int g0 = 0; g0 < total; g0 += kWave * NB) {
    uint4 v[NB];
    long long spins = 0;
    for (;;) {
#pragma unroll
      for (int u = 0; u < NB; u++)  // chunks past the end read as zero
        v[u] = __builtin_bit_cast(
            uint4, __builtin_amdgcn_raw_buffer_load_b128(r, (uint32_t)(g0 + u * kWave + lane) * 16u, 0, kCpolSC1));
      bool stale = false;
#pragma unroll
      for (int u = 0; u < NB; u++)
        if (g0 + u * kWave + lane < total) stale |= v[u].y != tag || v[u].w != tag;
      if (!__any(stale) || !link_retry(a, spins)) break;
    }
#pragma unroll
    for (int u = 0; u < NB; u++) {
      const int c = g0 + u * kWave + lane;
      if (c < total) *reinterpret_cast<uint2*>(sm.xs + c * 4) = make_uint2(v[u].x, v[u].z);
    }
  }
}

// RMSNorm weights of one sync-wave lane for K <= 4096, loaded before the poll
// (they never depend on the event).
struct NormRegs {
  uint4 g[8];
};

__device__ __forceinline__ void load_norm(NormRegs& nr, OpRef op, int lane) {
#pragma unroll
  for (int j = 0; j < 8; j++) {
    int c = (lane + kWave * j) * 8;
    nr.g[j] = c < op.K ? ldg16(op.norm + c) : make_uint4(0, 0, 0, 0);
  }
}

// Sync wave, after staging all of K: x * (rsqrt(mean(x^2) + eps) * w) rounded
// to bf16 (rmsnorm.cuh:120-124), in place.
__device__ __forceinline__ void norm_x(OpRef op, int T, int KB, Shared& sm, const NormRegs& nr, bool have_nr,
                                       int lane) {
  const int K = op.K;
  for (int b = 0; b < T; b++) {
    float ss = 0.f;
    for (int c = lane * 8; c < K; c += kWave * 8) {
      uint4 v = *reinterpret_cast<const uint4*>(&sm.xs[b * KB + xs_swz(b, c)]);
      uint32_t w4[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
      for (int e = 0; e < 4; e++) {
        float lo = lo16<DT_BF16>(w4[e]), hi = hi16<DT_BF16>(w4[e]);
        ss += lo * lo + hi * hi;
      }
    }
    ss = wave_sum(ss);
    const float r = rsqrtf(ss / (float)K + op.eps);
    for (int j = 0; lane * 8 + j * kWave * 8 < K; j++) {
      const int c = (lane + kWave * j) * 8;
      uint4 g;
      if (have_nr) {
        g = nr.g[0];
#pragma unroll
        for (int q = 1; q < 8; q++)
          if (j == q) g = nr.g[q];
      } else {
        g = ldg16(op.norm + c);
      }
      uint4 v = *reinterpret_cast<const uint4*>(&sm.xs[b * KB + xs_swz(b, c)]);
      uint32_t xv[4] = {v.x, v.y, v.z, v.w}, gv[4] = {g.x, g.y, g.z, g.w}, o[4];
#pragma unroll
      for (int e = 0; e < 4; e++) {
        float lo = lo16<DT_BF16>(xv[e]) * (r * lo16<DT_BF16>(gv[e]));
        float hi = hi16<DT_BF16>(xv[e]) * (r * hi16<DT_BF16>(gv[e]));
        o[e] = pack2<DT_BF16>(lo, hi);
      }
      *reinterpret_cast<uint4*>(&sm.xs[b * KB + xs_swz(b, c)]) = make_uint4(o[0], o[1], o[2], o[3]);
    }
  }
}

// One wave: row b of the staged activations (all of K <= 4096 in one
// block) times rsqrt(mean(x^2) + eps) * gamma (gamma staged in attn_p),
// rounded to bf16, in place -- the arithmetic of norm_x, with every LDS read
// of the row in flight at once.
__device__ __forceinline__ void norm_row(OpRef op, int b, int KB, Shared& sm, int lane, float eps) {
  // (a latency chain on the path from the input's arrival to the weight
  // stream: every LDS read is issued before any is waited for, addresses are
  // clamped instead of branched around, and the sum of squares is reduced in
  // registers)
  const int K = op.K;
  const uint16_t* gam = reinterpret_cast<const uint16_t*>(&sm.attn_p[0][0][0]);
  uint4 xv[8], gv[8];
  bool in[8];
#pragma unroll
  for (int j = 0; j < 8; j++) {
    const int c = (lane + kWave * j) * 8;
    in[j] = c < K;
    const int cc = in[j] ? c : 0;
    xv[j] = *reinterpret_cast<const uint4*>(&sm.xs[b * KB + xs_swz(b, cc)]);
    gv[j] = *reinterpret_cast<const uint4*>(gam + cc);
  }
  float ss = 0.f;
#pragma unroll
  for (int j = 0; j < 8; j++) {
    const uint32_t w4[4] = {xv[j].x, xv[j].y, xv[j].z, xv[j].w};
    float sj = 0.f;
#pragma unroll
    for (int e = 0; e < 4; e++) {
      const float lo = lo16<DT_BF16>(w4[e]), hi = hi16<DT_BF16>(w4[e]);
      sj += lo * lo + hi * hi;
    }
    ss += in[j] ? sj : 0.f;
  }
  ss = wave_sum_regs(ss);
  const float r = rsqrtf(ss / (float)K + eps);
#pragma unroll
  for (int j = 0; j < 8; j++) {
    const int c = (lane + kWave * j) * 8;
    const uint32_t xw[4] = {xv[j].x, xv[j].y, xv[j].z, xv[j].w}, gw[4] = {gv[j].x, gv[j].y, gv[j].z, gv[j].w};
    uint32_t o[4];
#pragma unroll
    for (int e = 0; e < 4; e++) {
      const float lo = lo16<DT_BF16>(xw[e]) * (r * lo16<DT_BF16>(gw[e]));
      const float hi = hi16<DT_BF16>(xw[e]) * (r * hi16<DT_BF16>(gw[e]));
      o[e] = pack2<DT_BF16>(lo, hi);
    }
    if (in[j]) *reinterpret_cast<uint4*>(&sm.xs[b * KB + xs_swz(b, c)]) = make_uint4(o[0], o[1], o[2], o[3]);
  }
}

// Row 0 (all of K <= 4096 in one block) normalized by the 8 waves together:
// wave w takes columns [512 w, 512 w + 512), one 16-byte chunk per lane; the
// sums of squares meet in LDS.  Same arithmetic as norm_row.
__device__ __forceinline__ void norm_row_split(OpRef op, int KB, Shared& sm, int wave, int lane, float eps) {
  const int K = op.K;
  const uint16_t* gam = reinterpret_cast<const uint16_t*>(&sm.attn_p[0][0][0]);
  const int c = (wave * kWave + lane) * 8;
  const bool in = c < K;
  const int cc = in ? c : 0;
  const uint4 xv = *reinterpret_cast<const uint4*>(&sm.xs[xs_swz(0, cc)]);
  const uint4 g = *reinterpret_cast<const uint4*>(gam + cc);
  const uint32_t xw[4] = {xv.x, xv.y, xv.z, xv.w}, gw[4] = {g.x, g.y, g.z, g.w};
  float s = 0.f;
#pragma unroll
  for (int e = 0; e < 4; e++) {
    const float lo = lo16<DT_BF16>(xw[e]), hi = hi16<DT_BF16>(xw[e]);
    s += lo * lo + hi * hi;
  }
  s = wave_sum_regs(in ? s : 0.f);
  if (lane == 0) sm.red[wave] = s;
  lds_sync();
  float ss = 0.f;
#pragma unroll
  for (int w = 0; w < PK_WAVES; w++) ss += sm.red[w];
  const float r = rsqrtf(ss / (float)K + eps);
  uint32_t o[4];
#pragma unroll
  for (int e = 0; e < 4; e++) {
    const float lo = lo16<DT_BF16>(xw[e]) * (r * lo16<DT_BF16>(gw[e]));
    const float hi = hi16<DT_BF16>(xw[e]) * (r * hi16<DT_BF16>(gw[e]));
    o[e] = pack2<DT_BF16>(lo, hi);
  }
  if (in) *reinterpret_cast<uint4*>(&sm.xs[xs_swz(0, c)]) = make_uint4(o[0], o[1], o[2], o[3]);
  lds_sync();  // row normalized
}

// Sync wave: one-lane event poll (the watchdog exits through sm.flag).
__device__ bool poll_event_sync(const KernelArgs& a, const TaskDesc& t, int task_id, Shared& sm) {
  if (tix() == SYNC_T0) {
    int ok = 1;
    if (t.wait_event >= 0) {
      const uint32_t need = (uint32_t)t.wait_count * a.epoch;
      long long spins = 0;
      for (;;) {
        const uint32_t v = __hip_atomic_load(gptr(&a.events[t.wait_event]), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        if (spins == 0 && a.profile) gptr(a.profile)[(size_t)task_id * 8 + 7] = now_10ns();  // first poll
        if ((int32_t)(v - need) >= 0) break;
        if ((spins & 255) == 255 && aborted(a)) { ok = 0; break; }
        if (++spins > a.spin_limit) {
          __hip_atomic_store(gptr(a.meta.status + 2), task_id, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
          __hip_atomic_store(gptr(a.meta.status), 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
          ok = 0;
          break;
        }
        __builtin_amdgcn_s_sleep(2);
      }
    }
    if (a.profile) gptr(a.profile)[(size_t)task_id * 8 + 1] = now_10ns();
    sm.flag = ok;
  }
  __builtin_amdgcn_wave_barrier();
  return __builtin_amdgcn_readfirstlane(sm.flag) != 0;  // lane 0 wrote it; LDS ops of a wave are in order
}

// Sum over the 64 lanes with DPP row operations (a handful of instructions,
// no LDS crossbar); the result is read from the last lane.
template <int CTRL, int ROW_MASK = 0xf>
__device__ __forceinline__ float dpp_term(float v) {
  return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, ROW_MASK, 0xf, false));
}
__device__ __forceinline__ float wave_sum_dpp(float v) {
  v += dpp_term<0xb1>(v);         // quad_perm [1,0,3,2]
  v += dpp_term<0x4e>(v);         // quad_perm [2,3,0,1]
  v += dpp_term<0x141>(v);        // row_half_mirror: 8-lane sums
  v += dpp_term<0x140>(v);        // row_mirror: 16-lane sums in every lane
  v += dpp_term<0x142, 0xa>(v);   // row_bcast:15 -> rows 1, 3
  v += dpp_term<0x143, 0xc>(v);   // row_bcast:31 -> rows 2, 3
  return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 63));
}

// Adds a compute wave's per-token partial sums into its LDS slot and clears
// them: a plain wave sum for one token; a reduce-scatter (10 shuffles) for 8.
template <int TM>
__device__ __forceinline__ void flush_acc(float (&acc)[TM], float* slot, int lane) {
  if constexpr (TM == 1) {
    const float v = wave_sum_dpp(acc[0]);
    if (lane == 0) slot[0] += v;
    acc[0] = 0.f;
  } else {
    static_assert(TM == 8, "token tiles of 1 or 8");
    const bool h32 = lane & 32, h16 = lane & 16, h8 = lane & 8;
    float a4[4], a2[2];
#pragma unroll
    for (int i = 0; i < 4; i++) a4[i] = (h32 ? acc[i + 4] : acc[i]) + __shfl_xor(h32 ? acc[i] : acc[i + 4], 32, kWave);
#pragma unroll
    for (int i = 0; i < 2; i++) a2[i] = (h16 ? a4[i + 2] : a4[i]) + __shfl_xor(h16 ? a4[i] : a4[i + 2], 16, kWave);
    float v = (h8 ? a2[1] : a2[0]) + __shfl_xor(h8 ? a2[0] : a2[1], 8, kWave);
    v += __shfl_xor(v, 4, kWave);
    v += __shfl_xor(v, 2, kWave);
    v += __shfl_xor(v, 1, kWave);
    if ((lane & 7) == 0) slot[(h32 ? 4 : 0) + (h16 ? 2 : 0) + (h8 ? 1 : 0)] += v;
#pragma unroll
    for (int i = 0; i < TM; i++) acc[i] = 0.f;
  }
}

// Number of staged K blocks: the fewest equal blocks of whole 512-element
// chunks whose activations fit the staging buffer -- or, when one block does
// not hold all of K, a quarter of it (QUAD: blocks rotate through four
// buffers, loaded straight into LDS up to three blocks ahead) or half of it
// (the 16-token RMSNorm ops, which scale rows on their way in: blocks
// alternate between two halves, block kb + 1 staged while kb is consumed).
__host__ __device__ __forceinline__ int gemv_blocks(int NC, int TM, bool quad) {
  int maxc = (XS_ELEMS / TM) >> 9;
  if (NC > maxc) maxc = quad ? maxc >> 2 : maxc >> 1;
  if (maxc < 1) maxc = 1;
  int nkb = (NC + maxc - 1) / maxc;
  while (NC % nkb) nkb++;
  return nkb;
}
constexpr int XS_HALF = XS_ELEMS / 2;     // second staging buffer (multi-block K)
constexpr int XS_QUARTER = XS_ELEMS / 4;  // QUAD staging buffers

// 16 bytes per lane from a buffer straight into LDS (lane l's data lands at
// lds_block + 16 l, lds_block wave-uniform), agent-coherent (sc1); an offset
// past the buffer writes zeros.  Inline assembly, so the compiler inserts no
// waits of its own for these loads: the sync wave orders them itself
// (s_waitcnt vmcnt, then the barrier that publishes the block).
__device__ __forceinline__ void bload_lds16_sc1(__amdgpu_buffer_rsrc_t r, uint32_t off, void* lds_block) {
  const uint32_t lds = __builtin_amdgcn_readfirstlane(
      (uint32_t)(uintptr_t)(__attribute__((address_space(3))) char*)(lds_block));
  asm volatile("s_mov_b32 m0, %1\n\tbuffer_load_dwordx4 %0, %2, 0 offen sc1 lds"
               :
               : "v"(off), "s"(lds), "s"(r)
               : "memory", "m0");
}
template <int N>
__device__ __forceinline__ void wait_vmcnt_le() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4) | (15 << 8));
}
// s_waitcnt vmcnt(n) for a wave-uniform n in {0, 8, 16, 24, 32, 40, 48}
// (blocks still allowed in flight x loads per block); other values round down
__device__ __forceinline__ void wait_dma(int n) {
  if (n >= 48) wait_vmcnt_le<48>();
  else if (n >= 40) wait_vmcnt_le<40>();
  else if (n >= 32) wait_vmcnt_le<32>();
  else if (n >= 24) wait_vmcnt_le<24>();
  else if (n >= 16) wait_vmcnt_le<16>();
  else if (n >= 8) wait_vmcnt_le<8>();
  else wait_vmcnt_le<0>();
}

// Sync wave, QUAD multi-block input: block [k0, k0 + KB) of rows [0, TM)
// into the staging buffer at xs + xoff by direct-to-LDS loads, one
// instruction per row and 512 columns (TM KB / 512 <= 16 in all).  LDS chunk
// p of row b receives global chunk p ^ b (the xs_swz layout); rows >= T
// read as zero.
template <int TM>
__device__ __forceinline__ void stage_x_dma(OpRef op, int T, int KB, int k0, Shared& sm, int lane, int xoff) {
  const int nrec = __builtin_amdgcn_readfirstlane((int)((size_t)T * op.x_ld * 2));
  const __amdgpu_buffer_rsrc_t r =
      __builtin_amdgcn_make_buffer_rsrc(const_cast<uint16_t*>(op.x), 0, nrec, 0x00020000);
  const int G = KB >> 9;  // 512-column groups per row (1 or 2)
#pragma unroll
  for (int b = 0; b < TM; b++)
    for (int g = 0; g < G; g++) {
      const uint32_t off = (uint32_t)((b * op.x_ld + k0 + (g * 64 + (lane ^ b)) * 8) * 2);
      bload_lds16_sc1(r, off, sm.xs + xoff + b * KB + g * 512);
    }
}

// 16-token RMSNorm ops, all 8 waves: block [k0, k0 + KB) of rows [0, TM),
// landed raw in the staging buffer at xs + xoff, scaled in place to
// x * (r_b * gamma) rounded to bf16 (the values stage_x<16, true> writes),
// with r_b from row_rms_coop (attn_ml) and gamma staged in attn_p.  Chunk
// position p of row b holds the row's chunk p ^ b (the xs_swz layout).
template <int TM>
__device__ __forceinline__ void norm_block_lds(Shared& sm, int KB, int k0, int xoff) {
  const uint16_t* const gam = reinterpret_cast<const uint16_t*>(&sm.attn_p[0][0][0]);
  const int cpr = KB >> 3;  // 8-element chunks per row
  for (int c = tix(); c < TM * cpr; c += PK_THREADS) {
    const int b = c / cpr, p = c - b * cpr;
    uint4* const ptr = reinterpret_cast<uint4*>(sm.xs + xoff + b * KB + p * 8);
    const uint4 x = *ptr;
    const uint4 g = *reinterpret_cast<const uint4*>(gam + k0 + ((p ^ b) << 3));
    const float rb = sm.attn_ml[0][b][0];
    const uint32_t xv[4] = {x.x, x.y, x.z, x.w}, gv[4] = {g.x, g.y, g.z, g.w};
    uint32_t o[4];
#pragma unroll
    for (int e = 0; e < 4; e++)
      o[e] = pack2<DT_BF16>(lo16<DT_BF16>(xv[e]) * (rb * lo16<DT_BF16>(gv[e])),
                            hi16<DT_BF16>(xv[e]) * (rb * hi16<DT_BF16>(gv[e])));
    *ptr = make_uint4(o[0], o[1], o[2], o[3]);
  }
}

// gamma (K <= 16384 elements) into attn_p, all 8 waves
__device__ __forceinline__ void stage_gamma_lds(OpRef op, Shared& sm) {
  uint16_t* const gam = reinterpret_cast<uint16_t*>(&sm.attn_p[0][0][0]);
  for (int e = tix() * 8; e < op.K; e += PK_THREADS * 8) *reinterpret_cast<uint4*>(gam + e) = ldg16(op.norm + e);
}

template <int TM, int EPI, bool PK = false>
__device__ __forceinline__ void task_gemv(const KernelArgs& a, const TaskDesc& t, int task_id, Shared& sm) {
  constexpr int RG = TM == 1 ? YR_PK_RING1 : TM == 8 ? YR_PK_RING8 : RING;  // weight loads in flight per compute lane
  constexpr bool SILU = EPI == EPI_SILU;
  constexpr bool NORM = EPI != EPI_LIN;
  OpRef op = op_of(a, t.op);
  const int K = op.K, R = t.rows;
  const float eps = op.eps;
  const int RT = SILU ? 2 * R : R;                 // weight rows streamed
  const int seg = SILU ? R : t.split_row;          // rows [0, seg) from w0, the rest from w1
  const int NC = K >> 9;                           // 512-element chunks per row
  // QUAD: multi-block inputs staged by direct loads into four buffers (the
  // 16-token RMSNorm ops then scale each block in LDS, see norm_block_lds)
  constexpr bool QUAD = TM > 1;
  constexpr bool NBLK = NORM && TM == 16;  // blocks normalized in LDS after they land
  const int nkb = TM == 1 ? 1 : gemv_blocks(NC, TM, QUAD);
  const bool dma = QUAD && nkb > 1;
  const int NCB = NC / nkb, KB = NCB << 9;         // chunks / elements per staged block
  // A unit is one 16-byte weight load per lane.  TM == 1: 512 elements of
  // one row (dot products on VALU); TM == 8 / 16: a 16-row x 32-column MFMA A
  // fragment (rows = a 16-row tile of the weight); the B operand is the
  // staged activations, one token per MFMA column (8 or 16 valid).
  constexpr bool MF = TM > 1;
  constexpr int USH = MF ? 5 : 9;                  // log2 columns per unit
  const int NT = MF ? (RT + 15) / 16 : RT;         // rows (TM == 1) or 16-row tiles
  const int UPR = KB >> USH;                       // units per row / tile and block
  const int U = NT * UPR;                          // units per block
  // wave index as a scalar: role branches are wave-uniform
  const int wave = __builtin_amdgcn_readfirstlane(tix() / kWave), lane = tix() % kWave;
  const bool is_sync = wave == CW;
  float* slots = reinterpret_cast<float*>(sm.outs);  // [(RT + CW) slots][TM]

  // this compute wave's unit range (the same in every block)
  const int u0 = (wave * U) / CW, u1 = ((wave + 1) * U) / CW;
  const int n = is_sync ? 0 : u1 - u0, total = n * nkb;
  const int row0 = u0 / UPR, c00 = u0 - row0 * UPR;
  // load cursor: unit l_i of the wave's stream, at row / tile l_row, unit
  // l_c of it; lrow points at lane's element of unit 0 of that row / tile in
  // the current block (TM == 8: lane's weight row 16 tile + lane % 16,
  // clamped to the last row, columns 8 (lane / 16) ..)
  const uint16_t* const w1b = t.w1 + lane * 8;
  auto row_ptr = [&](int row, int kb) __attribute__((always_inline)) -> const uint16_t* {
    if constexpr (MF) {
      const int r = min(row * 16 + lane % 16, RT - 1);
      return (r < seg ? t.w0 + (size_t)r * K : t.w1 + (size_t)(r - seg) * K) + (size_t)kb * KB + (lane / 16) * 8;
    } else {
      return (row < seg ? t.w0 + (size_t)row * K : t.w1 + (size_t)(row - seg) * K) + (size_t)kb * KB + lane * 8;
    }
  };
  int l_i = 0, l_ib = 0, l_kb = 0, l_row = row0, l_c = c00;
  const uint16_t* lrow = row_ptr(row0, 0);
  // packed weights (batch > 1): the host laid this task's weights out in
  // stream order, unit (block kb, unit u) at w0 + (kb U + u) 512 with lane
  // l's 16 bytes at + 8 l, so every load instruction reads 1 KiB contiguous
  // and a wave walks one sequential range per block.  The last tile's rows
  // past RT are padding: those lanes load nothing (out-of-range offset).
  constexpr bool packed = MF && PK;
  const __amdgpu_buffer_rsrc_t prs =
      __builtin_amdgcn_make_buffer_rsrc(const_cast<uint16_t*>(t.w0), 0, packed ? nkb * U * 1024 : 0, 0x00020000);
  const bool last_ok = (NT - 1) * 16 + lane % 16 < RT;  // this lane's row of the last tile exists
  uint32_t poff = (uint32_t)u0 * 1024u + lane * 16;
  int p_tile = row0, p_c = c00;
  uint4 ring[RG];
  auto issue = [&](uint4& dst) __attribute__((always_inline)) {
    if constexpr (packed) {
      if (l_i < total) {
        dst = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(
                                            prs, p_tile < NT - 1 || last_ok ? poff : 0xfffffff0u, 0, 0));
        l_i++;
        poff += 1024u;
        if (++p_c == UPR) {
          p_c = 0;
          p_tile++;
        }
        if (++l_ib == n) {
          l_ib = 0;
          poff += (uint32_t)(U - n) * 1024u;
          p_tile = row0;
          p_c = c00;
        }
      }
      return;
    }
    if (l_i < total) {
      dst = ldg16(lrow + (l_c << USH));
      l_i++;
      if (++l_c == UPR) {
        l_c = 0;
        l_row++;
        if constexpr (MF) lrow = row_ptr(l_row, l_kb);
        else lrow = l_row == seg ? w1b + (size_t)l_kb * KB : lrow + K;
      }
      if (TM > 1 && ++l_ib == n) {
        l_ib = 0;
        l_kb++;
        l_row = row0;
        l_c = c00;
        lrow = row_ptr(row0, l_kb);
      }
    }
  };
#pragma unroll
  for (int s = 0; s < RG; s++) issue(ring[s]);

  if (is_sync) {
    // ---------------- sync wave: inputs
    const bool same_op = sm.last_op == t.op && nkb == 1;  // this op's inputs are already staged
    int T = sm.last_T;
    if (!same_op) {
      NormRegs nr;
      // (16-token batches: K does not fit one staged block; rows are
      // normalized while they are staged, see row_rms_coop / stage_x_coop_nrm / stage_x<.., true>)
      const bool pre = NORM && TM != 16 && K <= 4096;
      if (pre) load_norm(nr, op, lane);
      // a link input is validated word by word: no event poll (measured
      // faster than polling the producers' counter first)
      if ((op.flags & OPF_X_LL) || poll_event_sync(a, t, task_id, sm)) {
        T = active_tokens(a, op);
        if (TM == 1 && (op.flags & OPF_X_LL)) {
          stage_x_link(a, op, KB, 0, sm, lane);
          if (a.profile && lane == 0) gptr(a.profile)[(size_t)task_id * 8 + 1] = now_10ns();  // inputs valid
        } else if (dma) {
          // blocks 0..3 straight into the four buffers; block 0 lands before [X]
          const int ahead = nkb - 1 < 3 ? nkb - 1 : 3;
          for (int j = 0; j <= ahead; j++) stage_x_dma<TM>(op, T, KB, j * KB, sm, lane, j * XS_QUARTER);
          wait_dma(ahead * TM * (KB >> 9));
          if (NBLK && lane == 0) sm.coop_stage = 3;  // row factors, then block 0 scaled, by all waves
        } else if (TM > 1 && !(NORM && !pre)) {
          if (lane == 0) sm.coop_stage = 1;  // block 0 staged by all waves after [X]
        } else if constexpr (NORM && TM == 16) {
          // row factors and block 0 by all waves after [X]
          if (lane == 0) sm.coop_stage = 2;
        } else {
          stage_x<TM>(op, T, KB, 0, sm, lane);
        }
        if (NORM && MF && pre) {
          // batch > 1: gamma to LDS; every wave then normalizes one row
          uint16_t* gam = reinterpret_cast<uint16_t*>(&sm.attn_p[0][0][0]);
#pragma unroll
          for (int j = 0; j < 8; j++) {
            const int c = (lane + kWave * j) * 8;
            if (c < K) *reinterpret_cast<uint4*>(gam + c) = nr.g[j];
          }
          if (lane == 0) sm.norm_rows = T;
        } else if (NORM && TM == 1 && pre) {
          // one row: the same parallel form, gamma through attn_p
          uint16_t* gam = reinterpret_cast<uint16_t*>(&sm.attn_p[0][0][0]);
#pragma unroll
          for (int j = 0; j < 8; j++) {
            const int c = (lane + kWave * j) * 8;
            if (c < K) *reinterpret_cast<uint4*>(gam + c) = nr.g[j];
          }
          // normalized by all 8 waves after [X] (one wave alone spends ~1.5 us
          // issuing the row's arithmetic while the others wait)
          if (lane == 0) sm.norm_rows = T > 0 ? -1 : 0;
        } else if (NORM && TM != 16) {
          norm_x(op, T, KB, sm, nr, pre, lane);
        }
      }
    } else if (a.profile && lane == 0) {
      gptr(a.profile)[(size_t)task_id * 8 + 1] = now_10ns();
    }
    for (int i = lane; i < (MF ? (NT + CW) * 16 : RT + CW) * TM; i += kWave) slots[i] = 0.f;
    if (lane == 0 && (same_op || !(NORM && TM != 16 && K <= 4096))) sm.norm_rows = 0;
    if (lane == 0) {
      sm.last_T = T;
      sm.last_op = nkb == 1 ? t.op : -1;
    }
  }
  lds_sync();  // [X]: block 0 staged (or to be staged by all waves), slots cleared
  if (!sm.flag) return;
  const int T = sm.last_T;
  if constexpr (TM > 1) {
    const int cs = __builtin_amdgcn_readfirstlane(sm.coop_stage);  // workgroup-uniform
    if constexpr (NBLK) {
      if (cs == 3) {
        stage_gamma_lds(op, sm);
        row_rms_coop<TM>(op, T, sm, wave, lane);
        lds_sync();  // row factors in attn_ml, gamma in attn_p
        norm_block_lds<TM>(sm, KB, 0, 0);
        lds_sync();  // block 0 normalized
        if (tix() == 0) sm.coop_stage = 0;
      }
    }
    if constexpr (NORM && TM == 16) {
      if (cs == 2) {
        row_rms_coop<TM>(op, T, sm, wave, lane);
        lds_sync();  // row factors in attn_ml
        stage_x_coop_nrm<TM>(op, T, KB, sm, wave, lane);
        lds_sync();  // block 0 staged
        if (tix() == 0) sm.coop_stage = 0;
      }
    }
    if (cs == 1) {
      stage_x_coop<TM>(op, T, KB, sm, wave, lane);
      lds_sync();  // block 0 staged
      if (tix() == 0) sm.coop_stage = 0;
    }
  }
  if (a.profile && tix() == SYNC_T0) gptr(a.profile)[(size_t)task_id * 8 + 4] = now_10ns();
  if constexpr (NORM && MF) {
    const int nr = __builtin_amdgcn_readfirstlane(sm.norm_rows);
    if (nr > 0) {  // workgroup-uniform
      if (wave < nr) norm_row(op, wave, KB, sm, lane, eps);
      lds_sync();  // rows normalized
    }
  } else if constexpr (NORM && TM == 1) {
    if (__builtin_amdgcn_readfirstlane(sm.norm_rows) < 0) norm_row_split(op, KB, sm, wave, lane, eps);
  }

  if (is_sync) {
    if (dma) {
      // QUAD: block kb sits in buffer kb & 3; up to three blocks are in
      // flight ahead of the one the compute waves consume.  [Bkb] = block kb
      // landed (this wave's loads of it complete) and block kb - 1 consumed,
      // whose buffer then takes block kb + 3.
      const int L = TM * (KB >> 9);
      for (int kb = 1; kb < nkb; kb++) {
        const int after = (nkb - 1 < kb + 2 ? nkb - 1 : kb + 2) - kb;  // blocks issued after kb
        wait_dma(after * L);
        lds_sync();  // [Bkb]
        if constexpr (NBLK) {
          norm_block_lds<TM>(sm, KB, kb * KB, (kb & 3) * XS_QUARTER);
          lds_sync();  // [Nkb]: block kb normalized
        }
        if (kb + 3 < nkb) stage_x_dma<TM>(op, T, KB, (kb + 3) * KB, sm, lane, ((kb + 3) & 3) * XS_QUARTER);
      }
    } else {
      // multi-block K (16-token RMSNorm ops): block kb goes to half kb & 1
      // while the compute waves consume block kb - 1 from the other half;
      // barrier [Bkb] = block kb staged and block kb - 1 consumed
      for (int kb = 1; kb < nkb; kb++) {
        stage_x<TM, NORM && TM == 16>(op, T, KB, kb * KB, sm, lane, (kb & 1) * XS_HALF);
        lds_sync();  // [Bkb]
      }
    }
  } else if (n == 0) {
    for (int kb = 1; kb < nkb; kb++) {
      lds_sync();  // [Bkb]
      if (NBLK && dma) {
        norm_block_lds<TM>(sm, KB, kb * KB, (kb & 3) * XS_QUARTER);
        lds_sync();  // [Nkb]
      }
    }
  } else {
    // ---------------- compute waves: stream the unit range
    if constexpr (MF) {
      // C of tile tl: rows 16 tl + 4 (lane / 16) + i, token lane % 16 (< TM
      // valid); partial sums go to slot tile (tl + wave), so the tiles of
      // one wave never share slots with another wave's
      const int bt = lane % 16;
      const bool bok = bt < TM;
      const uint16_t* xrow = sm.xs + bt * KB;
      f32x4 acc = {0.f, 0.f, 0.f, 0.f};
      int tl = row0, c = c00, ib = 0, kb = 0;
      for (int g0 = 0; g0 < total; g0 += RG) {
#pragma unroll
        for (int s = 0; s < RG; s++) {
          if (g0 + s < total) {
            if (ib == n) {  // next staged block, in the other half
              ib = 0;
              tl = row0;
              c = c00;
              kb++;
              xrow = sm.xs + (dma ? (kb & 3) * XS_QUARTER : (kb & 1) * XS_HALF) + bt * KB;
              lds_sync();  // [Bkb]
              if (NBLK && dma) {
                norm_block_lds<TM>(sm, KB, kb * KB, (kb & 3) * XS_QUARTER);
                lds_sync();  // [Nkb]
              }
            }
            const uint4 w = ring[s];
            issue(ring[s]);
            const uint4 xv = bok ? *reinterpret_cast<const uint4*>(xrow + xs_swz(bt, (c << 5) + (lane / 16) * 8))
                                 : make_uint4(0, 0, 0, 0);
            acc = mfma_bf16(w, xv, acc);
            ++ib;
            if (++c == UPR || ib == n) {
              if (bok) {
                float* sl = slots + ((tl + wave) * 16 + 4 * (lane / 16)) * TM + bt;
#pragma unroll
                for (int i = 0; i < 4; i++) sl[i * TM] += acc[i];
              }
              acc = f32x4{0.f, 0.f, 0.f, 0.f};
              if (c == UPR) {
                c = 0;
                tl++;
              }
            }
          }
        }
      }
    } else {
    float acc[TM];
#pragma unroll
    for (int b = 0; b < TM; b++) acc[b] = 0.f;
    int row = row0, c = c00, ib = 0;
    for (int g0 = 0; g0 < total; g0 += RG) {
#pragma unroll
      for (int s = 0; s < RG; s++) {
        if (g0 + s < total) {
          if (TM > 1 && ib == n) {  // (batch 1 stages all of K at once)
            ib = 0;
            row = row0;
            c = c00;
            lds_sync();
          }
          const uint4 w = ring[s];
          issue(ring[s]);
          const uint16_t* xb = sm.xs + (c << 9) + lane * 8;
#pragma unroll
          for (int b = 0; b < TM; b++) {
            const uint4 xv = *reinterpret_cast<const uint4*>(xb + b * KB);
            float v = acc[b];
            v = dot2<DT_BF16>(w.x, xv.x, v);
            v = dot2<DT_BF16>(w.y, xv.y, v);
            v = dot2<DT_BF16>(w.z, xv.z, v);
            v = dot2<DT_BF16>(w.w, xv.w, v);
            acc[b] = v;
          }
          ++ib;
          if (++c == NCB || ib == n) {
            flush_acc<TM>(acc, slots + (row + wave) * TM, lane);
            if (c == NCB) {
              c = 0;
              row++;
            }
          }
        }
      }
    }
    }
  }
  lds_sync();  // [O]: every partial sum is in its slot
  if (a.profile && tix() == SYNC_T0) gptr(a.profile)[(size_t)task_id * 8 + 5] = now_10ns();
  if (!is_sync) {
    // [E]: the sync wave's output stores go into the CU's memory queue ahead
    // of this wave's next-task weight loads (behind ~100 KiB of loads they
    // became visible to the consumers microseconds later)
    lds_sync();
    return;
  }

  // ---------------- sync wave: epilogue, stores, publish
  // value of weight row j for token b: its slots, in wave order
  auto rowval = [&](int j, int b) __attribute__((always_inline)) -> float {
    const int tj = MF ? j / 16 : j;
    const int wlo = ((tj * UPR + 1) * CW - 1) / U, whi = ((tj * UPR + UPR) * CW - 1) / U;
    float v = 0.f;
    for (int w = wlo; w <= whi; w++) v += slots[(MF ? (tj + w) * 16 + j % 16 : j + w) * TM + b];
    return v;
  };
  float* vals = &sm.attn_p[0][0][0];  // argmax: bf16-rounded logits [T][R]
  // (token, column pair) items, four per lane per round: the residual loads
  // of a round are all in flight before any is used
  const int NP = R / 2, tot = T * NP;
  const bool resid = !SILU && (op.flags & OPF_RESIDUAL);
  constexpr int KR = TM == 1 ? 1 : 4;  // items per lane and round
  for (int i0 = 0; i0 < tot; i0 += KR * kWave) {
    uint32_t rw[KR];
#pragma unroll
    for (int k = 0; k < KR; k++) rw[k] = 0u;
    if (resid) {
#pragma unroll
      for (int k = 0; k < KR; k++) {
        const int idx = i0 + k * kWave + lane;
        if (idx < tot) {
          const int b = idx / NP, p = idx - b * NP;
          const size_t re = (size_t)b * op.res_ld + t.row0 + 2 * p;
          rw[k] = op.flags & OPF_RES_LL ? link_load(a, op.residual, re, link_tag(a, op.res_src))
                                        : ld_agent_u32(op.residual + re);
        }
      }
    }
#pragma unroll
    for (int k = 0; k < KR; k++) {
      const int idx = i0 + k * kWave + lane;
      if (idx < tot) {
        const int b = idx / NP, p = idx - b * NP;
        float v0, v1;
        if constexpr (SILU) {
          // silu_mul.cuh:31-40 on the bf16 gate/up results
          float g0 = round_to<DT_BF16>(rowval(2 * p, b)), g1 = round_to<DT_BF16>(rowval(2 * p + 1, b));
          float x0 = round_to<DT_BF16>(rowval(R + 2 * p, b)), x1 = round_to<DT_BF16>(rowval(R + 2 * p + 1, b));
          v0 = round_to<DT_BF16>(g0 / (1.0f + expf(-g0))) * x0;
          v1 = round_to<DT_BF16>(g1 / (1.0f + expf(-g1))) * x1;
        } else {
          v0 = rowval(2 * p, b) + (resid ? lo16<DT_BF16>(rw[k]) : 0.f);
          v1 = rowval(2 * p + 1, b) + (resid ? hi16<DT_BF16>(rw[k]) : 0.f);
        }
        const uint32_t packed = pack2<DT_BF16>(v0, v1);
        const size_t oe = (size_t)b * op.out_ld + t.row0 + 2 * p;
        if (op.flags & OPF_OUT_LL) link_store(op.out, oe, packed, link_tag(a, t.op));
        else st_agent_u32(op.out + oe, packed);
        if (EPI == EPI_ARGMAX) {
          vals[b * R + 2 * p] = lo16<DT_BF16>(packed);  // argmax runs on the bf16 logits
          vals[b * R + 2 * p + 1] = hi16<DT_BF16>(packed);
        }
      }
    }
  }
  lds_sync();  // [E]
  if constexpr (EPI == EPI_ARGMAX) {
    // local (value, index) maximum per token over this task's valid rows;
    // lowest index wins ties (torch.argmax semantics)
    __builtin_amdgcn_wave_barrier();
    const int lim = op.vocab - t.row0 < R ? op.vocab - t.row0 : R;
    for (int b = 0; b < T; b++) {
      float best = -INFINITY;
      int bi = 0x7fffffff;
      for (int i = lane; i < lim; i += kWave) {
        float v = vals[b * R + i];
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
      last = __hip_atomic_fetch_add(gptr(&a.tickets[op.ticket_base]), 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) ==
             (uint32_t)(t.i1 - 1);
    last = __shfl(last, 0, kWave);
    if (last) {
      if (lane == 0) __hip_atomic_store(gptr(&a.tickets[op.ticket_base]), 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      // reduce every task's record; task order = column order
      for (int b = 0; b < T; b++) {
        float best = -INFINITY;
        int bi = 0x7fffffff;
        // 4 records in flight per lane (the max / lowest-index rule does not
        // depend on the order records are compared in)
        for (int k0 = lane; k0 < t.i1; k0 += 4 * kWave) {
          float v[4];
          int ix[4];
#pragma unroll
          for (int j = 0; j < 4; j++) {
            const int k = k0 + j * kWave;
            const float* rec = a.scratch + op.scratch_off + ((size_t)k * op.max_tokens + b) * 2;
            v[j] = k < t.i1 ? ld_agent(rec) : -INFINITY;
            ix[j] = k < t.i1 ? __float_as_int(ld_agent(rec + 1)) : -1;
          }
#pragma unroll
          for (int j = 0; j < 4; j++)
            if (ix[j] >= 0 && (v[j] > best || (v[j] == best && ix[j] < bi))) { best = v[j]; bi = ix[j]; }
        }
#pragma unroll
        for (int o = 32; o > 0; o >>= 1) {
          float ov = __shfl_xor(best, o, kWave);
          int oi = __shfl_xor(bi, o, kWave);
          if (ov > best || (ov == best && oi < bi)) { best = ov; bi = oi; }
        }
        if (lane == 0)
          __hip_atomic_store(gptr(reinterpret_cast<uint64_t*>(op.tokens_out + b)),
                             (uint64_t)(int64_t)(bi == 0x7fffffff ? -1 : bi), __ATOMIC_RELAXED,
                             __HIP_MEMORY_SCOPE_AGENT);
      }
    }
  }
  if (!(op.flags & OPF_OUT_LL)) wait_vm();  // link outputs are checked by their readers
  if (a.profile && lane == 0) gptr(a.profile)[(size_t)task_id * 8 + 6] = now_10ns();
  if (lane == 0 && t.trigger_event >= 0) {
    __hip_atomic_fetch_add(gptr(&a.events[t.trigger_event]), 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
}

// ------------------------------------------------------------ attention
// One task = (request r, kv head h, split s).  Cached positions [0, base) are
// divided between the splits; the last split also handles the new tokens
// (RoPE, append to the paged cache, causal mask), as the reference does in
// multitoken_paged_attention_4_16.cuh:227-560.  Query rows = token j * G + g
// (<= 16) in one MFMA 16x16x32 row block.

// RoPE (rotate-half, rotary_embedding.cuh:22-81) of one head vector held as
// four 8-element chunks per lane: chunk q covers d = 32 q + 8 (lane / 16).
// The rotate-half partner of chunk q (d +- D/2) is chunk (q + 2) % 4 of the
// same lane, so one load per chunk suffices.  Loads and arithmetic are split
// so that a wave can have several vectors in flight before it waits.
struct RopeVec {
  uint4 x[4], c[4], s[4];
};
// cos/sin of one position from a [cos 128 | sin 128] row staged in LDS
__device__ __forceinline__ void rope_tab_lds(RopeVec& v, const uint16_t* row, int lane) {
#pragma unroll
  for (int q = 0; q < 4; q++) {
    const int d = 32 * q + (lane / 16) * 8;
    v.c[q] = *reinterpret_cast<const uint4*>(row + d);
    v.s[q] = *reinterpret_cast<const uint4*>(row + 128 + d);
  }
}
__device__ __forceinline__ void rope_apply(const RopeVec& v, uint4 (&out)[4], OpRef op) {
#pragma unroll
  for (int q = 0; q < 4; q++) {
    if (!op.cos_t) {
      out[q] = v.x[q];
      continue;
    }
    const uint4 x = v.x[q], y = v.x[(q + 2) & 3], c = v.c[q], sn = v.s[q];
    uint32_t xv[4] = {x.x, x.y, x.z, x.w}, yv[4] = {y.x, y.y, y.z, y.w}, cv[4] = {c.x, c.y, c.z, c.w},
             sv[4] = {sn.x, sn.y, sn.z, sn.w}, o[4];
    const float sg = q < 2 ? -1.f : 1.f;  // first half: x cos - x[d + D/2] sin
#pragma unroll
    for (int e = 0; e < 4; e++) {
      float lo = lo16<DT_BF16>(xv[e]) * lo16<DT_BF16>(cv[e]) + sg * lo16<DT_BF16>(yv[e]) * lo16<DT_BF16>(sv[e]);
      float hi = hi16<DT_BF16>(xv[e]) * hi16<DT_BF16>(cv[e]) + sg * hi16<DT_BF16>(yv[e]) * hi16<DT_BF16>(sv[e]);
      o[e] = pack2<DT_BF16>(lo, hi);
    }
    out[q] = make_uint4(o[0], o[1], o[2], o[3]);
  }
}

// qk-norm (multitoken_paged_attention_4_16.cuh:348-375 calling
// tasks/ampere/norm.cuh:21-126): one head row of 128 values is RMS-normalized
// with weights w[128] (eps from the op), each value rounded to bf16 before
// RoPE reads it.  Row layout of the q / k fragments above: four 8-element
// chunks per lane (d = 32 q + 8 (lane / 16)), the row's other 96 values in
// lanes lane ^ 16, ^ 32, ^ 48.  Every lane of the wave must call it.
__device__ __forceinline__ void qk_norm4(uint4 (&x)[4], const uint16_t* w, int lane, float eps) {
  float ss = 0.f;
#pragma unroll
  for (int q = 0; q < 4; q++) {
    const uint32_t v[4] = {x[q].x, x[q].y, x[q].z, x[q].w};
#pragma unroll
    for (int e = 0; e < 4; e++) {
      const float lo = lo16<DT_BF16>(v[e]), hi = hi16<DT_BF16>(v[e]);
      ss += lo * lo + hi * hi;
    }
  }
  ss += __shfl_xor(ss, 16, kWave);
  ss += __shfl_xor(ss, 32, kWave);
  const float rr = rsqrtf(ss * (1.f / 128.f) + eps);
#pragma unroll
  for (int q = 0; q < 4; q++) {
    const uint4 wq = ldg16(w + 32 * q + (lane / 16) * 8);
    const uint32_t v[4] = {x[q].x, x[q].y, x[q].z, x[q].w}, wv[4] = {wq.x, wq.y, wq.z, wq.w};
    uint32_t o[4];
#pragma unroll
    for (int e = 0; e < 4; e++)
      o[e] = pack2<DT_BF16>(lo16<DT_BF16>(v[e]) * (rr * lo16<DT_BF16>(wv[e])),
                            hi16<DT_BF16>(v[e]) * (rr * hi16<DT_BF16>(wv[e])));
    x[q] = make_uint4(o[0], o[1], o[2], o[3]);
  }
}
// 8 values of a row given 1 / rms: x * (rr * w), rounded to bf16
__device__ __forceinline__ uint4 qk_scale8(uint4 x, const uint16_t* w8, float rr) {
  const uint4 wq = ldg16(w8);
  const uint32_t v[4] = {x.x, x.y, x.z, x.w}, wv[4] = {wq.x, wq.y, wq.z, wq.w};
  uint32_t o[4];
#pragma unroll
  for (int e = 0; e < 4; e++)
    o[e] = pack2<DT_BF16>(lo16<DT_BF16>(v[e]) * (rr * lo16<DT_BF16>(wv[e])),
                          hi16<DT_BF16>(v[e]) * (rr * hi16<DT_BF16>(wv[e])));
  return make_uint4(o[0], o[1], o[2], o[3]);
}
__device__ __forceinline__ float sumsq8(uint4 x) {
  const uint32_t v[4] = {x.x, x.y, x.z, x.w};
  float ss = 0.f;
#pragma unroll
  for (int e = 0; e < 4; e++) {
    const float lo = lo16<DT_BF16>(v[e]), hi = hi16<DT_BF16>(v[e]);
    ss += lo * lo + hi * hi;
  }
  return ss;
}

template <int RMAX>
__device__ __forceinline__ void task_attention_body(const KernelArgs& a, const TaskDesc& t, int task_id, int slot,
                                                    Shared& sm) {
  OpRef op = op_of(a, t.op);
  constexpr int D = 128;
  const int r = t.i0, h = t.i1, s = t.i2, S = op.splits;
  const int G = op.num_q_heads / op.num_kv_heads;
  const int wave = __builtin_amdgcn_readfirstlane(tix() / kWave), lane = tix() % kWave;
  const BatchMeta& m = a.meta;
  // request geometry (the page table is written by the host or by the
  // previous launch's prepare_batch task), read at descriptor load when the
  // worker's table had room
  const int pe = __builtin_amdgcn_readfirstlane((int)sm.pre_of[__builtin_amdgcn_readfirstlane(slot)]);
  const bool have_pre = pe != kPreNone;
  AttnGeom gm;
  if (have_pre) {
    const AttnPre& P = sm.pre[pe];
    gm.t0 = __builtin_amdgcn_readfirstlane(P.t0);
    gm.nt = __builtin_amdgcn_readfirstlane(P.nt);
    gm.pb = __builtin_amdgcn_readfirstlane(P.pb);
    gm.np = __builtin_amdgcn_readfirstlane(P.np);
    gm.base = __builtin_amdgcn_readfirstlane(P.base);
    gm.c0 = __builtin_amdgcn_readfirstlane(P.c0);
    gm.c1 = __builtin_amdgcn_readfirstlane(P.c1);
  } else {
    gm = attn_geom(m, op, r, s);
  }
  const int t0 = gm.t0, nt = gm.nt, pb = gm.pb, np = gm.np, base = gm.base, c0 = gm.c0, c1 = gm.c1;
  const bool last = s == S - 1;
  const size_t tok_stride = (size_t)op.num_kv_heads * D;
  const float scale = 1.4426950408889634f / sqrtf((float)D);

  // cached positions: blocks of 64; compute wave w takes blocks w, w + CW, ...
  // (at most op.attn_blocks / CW each)
  const int nblk = (c1 - c0 + 63) / 64;
  uint4 kf[4][4], vf[16];
  // a 64-position block spans at most two pages (the builder fixes the page
  // at kPage positions).  Both page ids are read first, so no K/V load waits
  // on them; positions past c1 are clamped to c1 - 1 (finite data whose
  // scores are masked), so the 32 loads issue without branches.
  struct BlkAddr {
    const uint16_t *kA, *kB, *vA, *vB;
    int plast, pw0;
  };
  auto blk_addr = [&](int blk, bool pre_ids) __attribute__((always_inline)) -> BlkAddr {
    const int p0 = c0 + blk * 64;
    const int pg0 = p0 / kPage;
    int idA, idB;
    if (pre_ids) {
      idA = __builtin_amdgcn_readfirstlane(sm.pre[pe].id[2 * blk]);
      idB = __builtin_amdgcn_readfirstlane(sm.pre[pe].id[2 * blk + 1]);
    } else {
      idA = __builtin_amdgcn_readfirstlane(gptr(m.kv_indices)[pb + pg0]);
      idB = __builtin_amdgcn_readfirstlane(pg0 + 1 < np ? gptr(m.kv_indices)[pb + pg0 + 1] : idA);
    }
    const size_t page_elems = (size_t)kPage * tok_stride;
    BlkAddr ba;
    ba.kA = op.k_cache + (size_t)idA * page_elems + (size_t)h * D;
    ba.kB = op.k_cache + (size_t)idB * page_elems + (size_t)h * D;
    ba.vA = op.v_cache + (size_t)idA * page_elems + (size_t)h * D;
    ba.vB = op.v_cache + (size_t)idB * page_elems + (size_t)h * D;
    ba.plast = c1 - 1 - pg0 * kPage;  // last valid in-window offset
    ba.pw0 = p0 - pg0 * kPage;        // window offset of p0
    return ba;
  };
  auto load_k = [&](const BlkAddr& ba) __attribute__((always_inline)) {
#pragma unroll
    for (int j = 0; j < 4; j++) {
      int o = min(ba.pw0 + 16 * j + lane % 16, ba.plast);
      const uint16_t* src =
          (o >= kPage ? ba.kB : ba.kA) + (uint32_t)((o & (kPage - 1)) * (int)tok_stride) + (lane / 16) * 8;
#pragma unroll
      for (int q = 0; q < 4; q++) kf[j][q] = ldg16(src + 32 * q);
    }
  };
  auto load_v = [&](const BlkAddr& ba) __attribute__((always_inline)) {
#pragma unroll
    for (int i = 0; i < 16; i++) {
      int o = min(ba.pw0 + lane / 16 + 4 * i, ba.plast);
      vf[i] = ldg16((o >= kPage ? ba.vB : ba.vA) + (uint32_t)((o & (kPage - 1)) * (int)tok_stride) + (lane % 16) * 8);
    }
  };
  const bool fits = nt > 0 && nt * G <= 16 && nblk <= op.attn_blocks;
  if (!fits) {  // nothing to do / beyond one MFMA row block or the block budget
    if (!(op.flags & OPF_X_LL) && !wait_event(a, t, task_id, sm)) return;
    if (nt > 0 && tix() == 0)
      __hip_atomic_store(gptr(a.meta.status + 3), task_id + 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    signal_event(a, t);
    return;
  }
  // The sync wave (no cached block) reads q -- and in the last split the new
  // tokens' k / v -- applies RoPE, appends the new k / v to the cache and
  // stages the fragments in xs (free until the final wave merge), while the
  // compute waves' cached-block loads are already in flight.
  const bool newtok = last && wave == CW;
  uint4* const qst = reinterpret_cast<uint4*>(sm.xs);  // [4][64 lanes] q fragments (RoPE applied)
  uint4* const kst = qst + 4 * kWave;                  // [4][64] new k, MFMA B layout (RoPE applied)
  uint4* const vst = kst + 4 * kWave;                  // [4][64] new v rows lane / 16 + 4 i2
  const bool lk = (op.flags & OPF_X_LL) != 0;
  if (wave == CW) {
    // a link-tensor qkv is validated word by word: no event poll
    if (lk || poll_event_sync(a, t, task_id, sm)) {
      const int qrow = lane % 16, qj = qrow / G, qg = qrow % G;
      const bool qok = qrow < nt * G;
      const uint32_t xtag = lk ? link_tag(a, op.x_src) : 0u;
      // element offsets into qkv (plain or link tensor): row t0 + j, head column
      const size_t e_grp = (size_t)t0 * op.qkv_ld + (size_t)h * (G + 2) * D;
      const size_t e_q = e_grp + (size_t)qj * op.qkv_ld + (size_t)qg * D;
      const Link8 z8 = {make_uint4(0, 0, 0, 0), make_uint4(0, 0, 0, 0)};
      // new token i = lane % 16 (k, MFMA B layout) / lane / 16 + 4 i2 (v);
      // nt * G <= 16 keeps every new v row below i2 = 4
      const int ik = lane % 16;
      const size_t e_k = e_grp + (size_t)ik * op.qkv_ld + (size_t)G * D;
      Link8 qr[4], kr[4], vr[4];
      auto issue = [&]() __attribute__((always_inline)) {
#pragma unroll
        for (int q = 0; q < 4; q++) qr[q] = qok ? act8_issue(lk, op.x, e_q + 32 * q + (lane / 16) * 8) : z8;
        if (newtok) {
#pragma unroll
          for (int q = 0; q < 4; q++) kr[q] = ik < nt ? act8_issue(lk, op.x, e_k + 32 * q + (lane / 16) * 8) : z8;
#pragma unroll
          for (int i2 = 0; i2 < 4; i2++) {
            const int iv = lane / 16 + 4 * i2;
            vr[i2] = iv < nt ? act8_issue(lk, op.x,
                                          e_grp + (size_t)iv * op.qkv_ld + (size_t)(G + 1) * D + (lane % 16) * 8)
                             : z8;
          }
        }
      };
      auto stale = [&]() __attribute__((always_inline)) -> bool {
        bool st = false;
#pragma unroll
        for (int q = 0; q < 4; q++) st |= qok && !act8_ok(lk, qr[q], xtag);
        if (newtok) {
#pragma unroll
          for (int q = 0; q < 4; q++) st |= ik < nt && !act8_ok(lk, kr[q], xtag);
#pragma unroll
          for (int i2 = 0; i2 < 4; i2++) st |= lane / 16 + 4 * i2 < nt && !act8_ok(lk, vr[i2], xtag);
        }
        return __any(st);
      };
      issue();
      // [Q] (plain input): the q loads go into the CU's memory queue ahead of
      // the compute waves' cached-block loads (~200 KiB at batch 8)
      if (!lk) lds_sync();
      int pg_tok = 0;  // page of new token lane % 16
      if (newtok && qrow < nt)
        pg_tok = have_pre && qrow < 4 ? sm.pre[pe].pg_tok[qrow] : gptr(m.kv_indices)[pb + (base + qrow) / kPage];
      // RoPE tables of positions base .. base + nt - 1 ([pos][cos 128 | sin
      // 128]) in this wave's attn_p area
      uint16_t* const tabs = reinterpret_cast<uint16_t*>(&sm.attn_p[wave][0][0]);
      if (op.cos_t) {
        for (int c = lane; c < nt * 32; c += kWave) {
          const int pp = c / 32, tb = (c / 16) & 1, d = (c % 16) * 8;
          *reinterpret_cast<uint4*>(tabs + pp * 256 + tb * 128 + d) =
              ldg16((tb ? op.sin_t : op.cos_t) + (size_t)(base + pp) * D + d);
        }
      }
      long long spins = 0;
      while (stale() && link_retry(a, spins)) issue();  // re-read while any word is stale
      RopeVec qin;
      rope_tab_lds(qin, tabs + (qok ? qj : 0) * 256, lane);
#pragma unroll
      for (int q = 0; q < 4; q++) qin.x[q] = act8_data(lk, qr[q]);
      if (op.flags & OPF_QK_NORM) qk_norm4(qin.x, op.norm, lane, op.eps);
      uint4 qo[4];
      rope_apply(qin, qo, op);
#pragma unroll
      for (int q = 0; q < 4; q++) qst[q * kWave + lane] = qo[q];
      if (newtok) {
        const bool kok = ik < nt;
        RopeVec kin;
        rope_tab_lds(kin, tabs + (kok ? ik : 0) * 256, lane);
#pragma unroll
        for (int q = 0; q < 4; q++) kin.x[q] = act8_data(lk, kr[q]);
        if (op.flags & OPF_QK_NORM) qk_norm4(kin.x, op.k_norm, lane, op.eps);
        uint4 ko[4];
        rope_apply(kin, ko, op);
        auto tok_off = [&](int pg, int pos) __attribute__((always_inline)) -> size_t {
          return ((size_t)pg * kPage + pos % kPage) * tok_stride + (size_t)h * D;
        };
#pragma unroll
        for (int q = 0; q < 4; q++) {
          kst[q * kWave + lane] = ko[q];
          if (kok) *reinterpret_cast<uint4*>(op.k_cache + tok_off(pg_tok, base + ik) + 32 * q + (lane / 16) * 8) = ko[q];
        }
#pragma unroll
        for (int i2 = 0; i2 < 4; i2++) {
          const int iv = lane / 16 + 4 * i2;
          const int pgv = __shfl(pg_tok, iv & 15, kWave);
          const uint4 vv = act8_data(lk, vr[i2]);
          vst[i2 * kWave + lane] = vv;
          if (iv < nt) *reinterpret_cast<uint4*>(op.v_cache + tok_off(pgv, base + iv) + (lane % 16) * 8) = vv;
        }
      }
    }
    else if (!lk) {
      lds_sync();  // [Q] (the poll failed; nothing to issue)
    }
  }
  // prefetch the first cached block of this wave
  if (!lk && wave < CW) lds_sync();  // [Q]
  if (wave < nblk && wave < CW) {
    const BlkAddr ba = blk_addr(wave, have_pre);
    load_k(ba);
    load_v(ba);
  }
  lds_sync();  // q (and new k / v) staged
  if (!__builtin_amdgcn_readfirstlane(sm.flag)) return;
  uint4 qf[4];
#pragma unroll
  for (int q = 0; q < 4; q++) qf[q] = qst[q * kWave + lane];
  if (newtok) {
#pragma unroll
    for (int q = 0; q < 4; q++) {
      kf[0][q] = kst[q * kWave + lane];
      kf[1][q] = kf[2][q] = kf[3][q] = make_uint4(0, 0, 0, 0);
    }
#pragma unroll
    for (int i2 = 0; i2 < 16; i2++) vf[i2] = i2 < 4 ? vst[i2 * kWave + lane] : make_uint4(0, 0, 0, 0);
  }
  // profile: 5 = q (and new k / v) loaded and valid, 4 = waves merged,
  // 7 = arrival ticket taken, 6 = split merge written (last split only)
  if (a.profile && tix() == 0) gptr(a.profile)[(size_t)task_id * 8 + 5] = now_10ns();

  // per-wave online softmax state for rows 4*(lane/16)+i
  float m_i[4], l_i[4];
  float o_acc[RMAX][8];  // [query row][8 dims of this lane's d-chunk]
#pragma unroll
  for (int i = 0; i < 4; i++) { m_i[i] = -INFINITY; l_i[i] = 0.f; }
#pragma unroll
  for (int rr = 0; rr < RMAX; rr++)
#pragma unroll
    for (int e = 0; e < 8; e++) o_acc[rr][e] = 0.f;

  // one 64-position block: qk_softmax (uses kf) then pv (uses vf);
  // mask(p_local, row) -> visible
  auto qk_softmax = [&](int p0, int npos, bool causal_new) __attribute__((always_inline)) {
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
      mx = row16_max(mx);
      float mnew = fmaxf(m_i[i], mx);
      float alpha = mnew == -INFINITY ? 1.f : exp2f(m_i[i] - mnew);
      float ls = 0.f;
#pragma unroll
      for (int j = 0; j < 4; j++) {
        float p = mnew == -INFINITY ? 0.f : exp2f(sc[j][i] - mnew);
        ls += p;
        sm.attn_p[wave][row][16 * j + lane % 16] = p;
      }
      ls = row16_sum(ls);
      l_i[i] = l_i[i] * alpha + ls;
      m_i[i] = mnew;
      if ((lane % 16) == 0) sm.attn_ml[wave][row][0] = alpha;
    }
    __builtin_amdgcn_s_waitcnt(0xc07f);
    __builtin_amdgcn_wave_barrier();
  };
  auto pv = [&]() __attribute__((always_inline)) {
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

  // the compute waves' blocks: the next block's K loads go out once this
  // block's K is consumed, its V loads once this block's V is
  if (wave < CW) {
    // every block but the wave's last also loads its successor (loads stay
    // unconditional, so no register array is live twice)
    int blk = wave;
    for (; blk + CW < nblk; blk += CW) {
      const BlkAddr bn = blk_addr(blk + CW, false);
      qk_softmax(c0 + blk * 64, 64, false);
      // scheduling fences: the next block's loads must not move above the
      // uses of the registers they overwrite
      __builtin_amdgcn_sched_barrier(0);
      load_k(bn);
      __builtin_amdgcn_sched_barrier(0);
      pv();
      __builtin_amdgcn_sched_barrier(0);
      load_v(bn);
      __builtin_amdgcn_sched_barrier(0);
    }
    if (blk < nblk) {
      const int npos = (c1 - c0) - blk * 64;
      qk_softmax(c0 + blk * 64, npos < 64 ? npos : 64, false);
      pv();
    }
  }

  // new tokens: causal block on the sync wave of the last split
  if (newtok) {
    qk_softmax(base, nt, true);
    pv();
  }
  if (a.profile && tix() == 0) gptr(a.profile)[(size_t)task_id * 8 + 1] = now_10ns();  // wave 0 processed

  // sum o over the 4 lane groups (positions lane/16 + 4 i), then merge the
  // 8 waves: per row, (m, l) in LDS, o through LDS (xs reused as float)
#pragma unroll
  for (int rr = 0; rr < RMAX; rr++)
#pragma unroll
    for (int e = 0; e < 8; e++) {
      o_acc[rr][e] = add_xor32(add_xor16(o_acc[rr][e]));
    }
  float* o_lds = reinterpret_cast<float*>(sm.xs);  // [wave][16 rows][128]
  lds_sync();
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
  lds_sync();
  if (a.profile && tix() == 0) gptr(a.profile)[(size_t)task_id * 8 + 4] = now_10ns();
  // Split merge without an arrival ticket: every split but the last writes
  // its (O, m, l) record as tagged words {f32, tag of this launch and op}
  // (single-copy atomic 8-byte stores, nothing awaited); the last split --
  // which also appended the new tokens -- keeps its own partial in LDS,
  // re-reads the other records until every word carries this launch's tag,
  // and merges.  (An arrival ticket costs a store acknowledgement and an
  // atomic round trip on the chain before the merge can start.)
  const int rows = nt * G;
  const uint32_t rtag = link_tag(a, t.op);
  const int rec_words = op.rec_rows * (D + 2);  // [rows][D + 2] words per split
  uint64_t* const rec_base = reinterpret_cast<uint64_t*>(a.scratch + op.scratch_off) +
                             (((size_t)r * op.num_kv_heads + h) * S) * rec_words;
  float* const own = reinterpret_cast<float*>(sm.outs);  // last split: [rows][D] O, then [rows][2] (m, l)
  float* const own_ml = own + 16 * D;
  for (int idx = tix(); idx < rows * D; idx += PK_THREADS) {
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
    if (last) {
      own[rr * D + d] = O;
      if (d == 0) {
        own_ml[2 * rr] = M;
        own_ml[2 * rr + 1] = L;
      }
    } else {
      uint64_t* const rec = rec_base + (size_t)s * rec_words + rr * (D + 2);
      auto put = [&](int i, float v) __attribute__((always_inline)) {
        __hip_atomic_store(gptr(rec + i), (uint64_t)__float_as_uint(v) | ((uint64_t)rtag << 32), __ATOMIC_RELAXED,
                           __HIP_MEMORY_SCOPE_AGENT);
      };
      put(d, O);
      if (d == 0) {
        put(D, M);
        put(D + 1, L);
      }
    }
  }
  if (last) {
    lds_sync();  // own partial in outs
    // thread -> (unit = row x 4-float d chunk, lane j of P, P a power of 2):
    // lane j takes splits j, j + P, ... (the own partial is split S - 1) in
    // rounds of 4, all of a round's words loaded at once and re-read while
    // any is stale, folded into a running (m, l, o) in registers; the P lanes
    // of a unit are consecutive and combine by DPP.  No LDS round trips.
    const int tid = tix();
    const int units = rows * (D / 4);
    int P = 1;
    while (2 * P * units <= PK_THREADS) P *= 2;
    const int u = tid / P, j = tid % P;
    const bool act = u < units;
    const int rr = act ? u / (D / 4) : 0, d4 = act ? (u % (D / 4)) * 4 : 0;
    const __amdgpu_buffer_rsrc_t rsr = __builtin_amdgcn_make_buffer_rsrc(rec_base, 0, 0x7fffffff, 0x00020000);
    auto ld16 = [&](size_t word) __attribute__((always_inline)) -> uint4 {  // two tagged words
      return __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(rsr, (uint32_t)(word * 8), 0, kCpolSC1));
    };
    float m_run = -INFINITY, l_run = 0.f, o[4] = {0.f, 0.f, 0.f, 0.f};
    long long spins = 0;
    for (int s0 = j; s0 < S; s0 += 4 * P) {
      uint4 wo[4][2], wm[4];
      auto issue = [&]() __attribute__((always_inline)) {
#pragma unroll
        for (int q = 0; q < 4; q++) {
          const int s2 = s0 + q * P;
          const size_t base_w = (size_t)(act && s2 < S - 1 ? s2 : 0) * rec_words + rr * (D + 2);
          wo[q][0] = ld16(base_w + d4);
          wo[q][1] = ld16(base_w + d4 + 2);
          wm[q] = ld16(base_w + D);
        }
      };
      auto stale = [&]() __attribute__((always_inline)) -> bool {
        bool st = false;
#pragma unroll
        for (int q = 0; q < 4; q++)
          st |= act && s0 + q * P < S - 1 &&
                (wo[q][0].y != rtag || wo[q][0].w != rtag || wo[q][1].y != rtag || wo[q][1].w != rtag ||
                 wm[q].y != rtag || wm[q].w != rtag);
        return st;
      };
      issue();
      while (stale() && link_retry(a, spins)) issue();
#pragma unroll
      for (int q = 0; q < 4; q++) {
        const int s2 = s0 + q * P;
        if (act && s2 < S) {
          const bool mine = s2 == S - 1;
          const float ms = mine ? own_ml[2 * rr] : __uint_as_float(wm[q].x);
          const float ls = mine ? own_ml[2 * rr + 1] : __uint_as_float(wm[q].z);
          float os[4];
          if (mine) {
#pragma unroll
            for (int e = 0; e < 4; e++) os[e] = own[rr * D + d4 + e];
          } else {
            os[0] = __uint_as_float(wo[q][0].x);
            os[1] = __uint_as_float(wo[q][0].z);
            os[2] = __uint_as_float(wo[q][1].x);
            os[3] = __uint_as_float(wo[q][1].z);
          }
          const float mn = fmaxf(m_run, ms);
          const float a1 = m_run == -INFINITY ? 0.f : exp2f(m_run - mn);
          const float a2 = ms == -INFINITY ? 0.f : exp2f(ms - mn);
          l_run = l_run * a1 + ls * a2;
#pragma unroll
          for (int e = 0; e < 4; e++) o[e] = o[e] * a1 + os[e] * a2;
          m_run = mn;
        }
      }
    }
    if (a.profile && tid == 0) gptr(a.profile)[(size_t)task_id * 8 + 7] = now_10ns();  // records read
    // combine the P lanes of each unit
    float Mt = m_run;
#pragma unroll
    for (int k = 0; k < 4; k++)
      if ((2 << k) <= P) Mt = fmaxf(Mt, dpp_f(Mt, k));
    const float f = m_run == -INFINITY ? 0.f : exp2f(m_run - Mt);
    float lt = l_run * f;
#pragma unroll
    for (int e = 0; e < 4; e++) o[e] *= f;
#pragma unroll
    for (int k = 0; k < 4; k++)
      if ((2 << k) <= P) {
        lt += dpp_f(lt, k);
#pragma unroll
        for (int e = 0; e < 4; e++) o[e] += dpp_f(o[e], k);
      }
    if (act && j == 0) {
      const float inv = lt > 0.f ? 1.f / lt : 0.f;
      const int jt = rr / G, g = rr % G;
      const size_t oe = (size_t)(t0 + jt) * op.out_ld + (size_t)(h * G + g) * D + d4;
      const uint32_t lo = pack2<DT_BF16>(o[0] * inv, o[1] * inv), hi = pack2<DT_BF16>(o[2] * inv, o[3] * inv);
      if (op.flags & OPF_OUT_LL) {
        const uint32_t otag = link_tag(a, t.op);
        link_store(op.out, oe, lo, otag);
        link_store(op.out, oe + 2, hi, otag);
      } else {
        __hip_atomic_store(gptr(reinterpret_cast<uint64_t*>(op.out + oe)), (uint64_t)lo | ((uint64_t)hi << 32),
                           __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      }
    }
    if (a.profile && tix() == 0) gptr(a.profile)[(size_t)task_id * 8 + 6] = now_10ns();
  }
  signal_event(a, t, (op.flags & OPF_OUT_LL) != 0);
}

// Multi-token attention task: a request with more than 16 query rows per kv
// head (nt * G > 16: prefill / extend chunks), the case of
// multitoken_paged_attention_32_64.cuh:40-710.  Same task grid, split
// ranges and split records as the single-block body above, organised for
// rows instead of latency:
//   * the whole workgroup waits for the QKV event (plain tensors only: link
//     tensors exist only in batch-1 graphs, where nt * G <= 16);
//   * the last split stages the nt new tokens' k (RoPE applied) and v in LDS
//     and appends them to the paged cache;
//   * wave w takes the 16-row blocks w, w + 8, ... (row = token j * G + head
//     g): q with RoPE from the QKV rows, then every cached 64-position block
//     of the split (K / V from the cache) and, in the last split, the new
//     tokens from LDS under the causal mask (position base + i visible to
//     token j iff i <= j), with an online softmax; its rows' (o, m, l) go to
//     the split record;
//   * the last split task to arrive merges the records of all rows.
__device__ __forceinline__ void task_attention_mt(const KernelArgs& a, const TaskDesc& t, int task_id, Shared& sm) {
  OpRef op = op_of(a, t.op);
  constexpr int D = 128;
  const int r = t.i0, h = t.i1, s = t.i2, S = op.splits;
  const int G = op.num_q_heads / op.num_kv_heads;
  const int wave = __builtin_amdgcn_readfirstlane(tix() / kWave), lane = tix() % kWave;
  const BatchMeta& m = a.meta;
  if (!wait_event(a, t, task_id, sm)) return;
  const AttnGeom gm = attn_geom(m, op, r, s);
  const int t0 = gm.t0, nt = gm.nt, pb = gm.pb, np = gm.np, base = gm.base, c0 = gm.c0, c1 = gm.c1;
  const int R = nt * G;
  if (R > op.rec_rows || (op.flags & (OPF_X_LL | OPF_OUT_LL)) || nt > XS_ELEMS / (2 * D)) {
    if (tix() == 0) __hip_atomic_store(gptr(a.meta.status + 3), task_id + 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    signal_event(a, t);
    return;
  }
  const bool last = s == S - 1;
  const size_t tok_stride = (size_t)op.num_kv_heads * D;
  const float scale = 1.4426950408889634f / sqrtf((float)D);
  const size_t e_grp = (size_t)h * (G + 2) * D;  // this kv head's [q x G | k | v] columns of a qkv row
  uint16_t* const knew = sm.xs;                  // [nt][D] new k (RoPE applied)
  uint16_t* const vnew = sm.xs + (size_t)nt * D; // [nt][D] new v
  if (last) {
    for (int idx = tix(); idx < nt * 16; idx += PK_THREADS) {
      const int i = idx / 16, c = idx % 16, cp = (c + 8) & 15;  // 8-dim chunk and its rotate-half partner
      const uint16_t* row = op.x + (size_t)(t0 + i) * op.qkv_ld + e_grp;
      uint4 kx = ld_agent_u128(row + (size_t)G * D + 8 * c);
      uint4 kp = ld_agent_u128(row + (size_t)G * D + 8 * cp);
      const uint4 vv = ld_agent_u128(row + (size_t)(G + 1) * D + 8 * c);
      if (op.flags & OPF_QK_NORM) {
        // the row's 16 chunks sit in 16 consecutive lanes (idx % 16 = c)
        float ss = sumsq8(kx);
        ss += __shfl_xor(ss, 1, kWave);
        ss += __shfl_xor(ss, 2, kWave);
        ss += __shfl_xor(ss, 4, kWave);
        ss += __shfl_xor(ss, 8, kWave);
        const float rr = rsqrtf(ss * (1.f / 128.f) + op.eps);
        kx = qk_scale8(kx, op.k_norm + 8 * c, rr);
        kp = qk_scale8(kp, op.k_norm + 8 * cp, rr);
      }
      uint4 kr = kx;
      if (op.cos_t) {
        const int pos = base + i;
        const uint4 cv = ldg16(op.cos_t + (size_t)pos * D + 8 * c), sv = ldg16(op.sin_t + (size_t)pos * D + 8 * c);
        const uint32_t xv[4] = {kx.x, kx.y, kx.z, kx.w}, yv[4] = {kp.x, kp.y, kp.z, kp.w};
        const uint32_t cw[4] = {cv.x, cv.y, cv.z, cv.w}, sw[4] = {sv.x, sv.y, sv.z, sv.w};
        const float sg = c < 8 ? -1.f : 1.f;  // first half: x cos - x[d + D/2] sin
        uint32_t o[4];
#pragma unroll
        for (int e = 0; e < 4; e++) {
          const float lo = lo16<DT_BF16>(xv[e]) * lo16<DT_BF16>(cw[e]) + sg * lo16<DT_BF16>(yv[e]) * lo16<DT_BF16>(sw[e]);
          const float hi = hi16<DT_BF16>(xv[e]) * hi16<DT_BF16>(cw[e]) + sg * hi16<DT_BF16>(yv[e]) * hi16<DT_BF16>(sw[e]);
          o[e] = pack2<DT_BF16>(lo, hi);
        }
        kr = make_uint4(o[0], o[1], o[2], o[3]);
      }
      *reinterpret_cast<uint4*>(knew + (size_t)i * D + 8 * c) = kr;
      *reinterpret_cast<uint4*>(vnew + (size_t)i * D + 8 * c) = vv;
      const int pos = base + i;
      const int pg = gptr(m.kv_indices)[pb + pos / kPage];
      const size_t ce = ((size_t)pg * kPage + pos % kPage) * tok_stride + (size_t)h * D + 8 * c;
      *reinterpret_cast<uint4*>(op.k_cache + ce) = kr;
      *reinterpret_cast<uint4*>(op.v_cache + ce) = vv;
    }
  }
  lds_sync();  // new k / v staged

  const int rec_floats = op.rec_rows * (D + 2);
  // (records sized for the tagged words of the single-block body: 2 floats each)
  float* const rec_base = a.scratch + op.scratch_off + (((size_t)r * op.num_kv_heads + h) * S) * (2 * rec_floats);
  float* const rec = rec_base + (size_t)s * rec_floats;
  const int nblk = (c1 - c0 + 63) / 64;
  const int RB = (R + 15) / 16;
  float* const pw = &sm.attn_p[wave][0][0];   // P of this wave's row block [16][64]
  float* const aw = &sm.attn_ml[wave][0][0];  // per-row rescale factors [16][2]
  for (int rb = wave; rb < RB; rb += PK_WAVES) {
    // q of rows 16 rb + lane % 16 (MFMA A operand: 8 dims 32 q + 8 (lane / 16) per chunk), RoPE at base + j
    uint4 qf[4];
    {
      const int row = 16 * rb + lane % 16;
      const bool ok = row < R;
      const int j = ok ? row / G : 0, g = row % G;
      const uint16_t* src = op.x + (size_t)(t0 + j) * op.qkv_ld + e_grp + (size_t)g * D + (lane / 16) * 8;
      RopeVec qv;
#pragma unroll
      for (int q = 0; q < 4; q++) {
        qv.x[q] = ok ? ld_agent_u128(src + 32 * q) : make_uint4(0, 0, 0, 0);
        if (op.cos_t) {
          const size_t pe = (size_t)(base + j) * D + 32 * q + (lane / 16) * 8;
          qv.c[q] = ldg16(op.cos_t + pe);
          qv.s[q] = ldg16(op.sin_t + pe);
        }
      }
      if (op.flags & OPF_QK_NORM) qk_norm4(qv.x, op.norm, lane, op.eps);
      rope_apply(qv, qf, op);
    }
    float m_i[4], l_i[4], o_acc[16][8];
#pragma unroll
    for (int i = 0; i < 4; i++) { m_i[i] = -INFINITY; l_i[i] = 0.f; }
#pragma unroll
    for (int rr = 0; rr < 16; rr++)
#pragma unroll
      for (int e = 0; e < 8; e++) o_acc[rr][e] = 0.f;
    // one 64-position block: scores on MFMA against the K fragments (token
    // 16 jb + lane % 16), online softmax (P and the row rescale through
    // LDS), then P V on VALU against the V rows (token lane / 16 + 4 i2)
    auto block = [&](const uint4 (&kf)[4][4], const uint4 (&vf)[16], int npos, bool causal_new, int coff)
                     __attribute__((always_inline)) {
      f32x4 sc[4];
#pragma unroll
      for (int jb = 0; jb < 4; jb++) {
        f32x4 c = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int q = 0; q < 4; q++) c = mfma_bf16(qf[q], kf[jb][q], c);
        sc[jb] = c;
      }
#pragma unroll
      for (int i = 0; i < 4; i++) {
        const int rloc = 4 * (lane / 16) + i, row = 16 * rb + rloc;
        const int tj = row / G;
        float mx = -INFINITY;
#pragma unroll
        for (int jb = 0; jb < 4; jb++) {
          const int pl = 16 * jb + lane % 16;
          const bool vis = pl < npos && row < R && (!causal_new || coff + pl <= tj);
          const float v = vis ? sc[jb][i] * scale : -INFINITY;
          sc[jb][i] = v;
          mx = fmaxf(mx, v);
        }
        mx = row16_max(mx);
        const float mnew = fmaxf(m_i[i], mx);
        const float alpha = mnew == -INFINITY ? 1.f : exp2f(m_i[i] - mnew);
        float ls = 0.f;
#pragma unroll
        for (int jb = 0; jb < 4; jb++) {
          const float p = mnew == -INFINITY ? 0.f : exp2f(sc[jb][i] - mnew);
          ls += p;
          pw[rloc * 64 + 16 * jb + lane % 16] = p;
        }
        ls = row16_sum(ls);
        l_i[i] = l_i[i] * alpha + ls;
        m_i[i] = mnew;
        if ((lane % 16) == 0) aw[rloc * 2] = alpha;
      }
      __builtin_amdgcn_s_waitcnt(0xc07f);
      __builtin_amdgcn_wave_barrier();
#pragma unroll
      for (int rr = 0; rr < 16; rr++) {
        const float al = aw[rr * 2];
#pragma unroll
        for (int e = 0; e < 8; e++) o_acc[rr][e] *= al;
      }
#pragma unroll
      for (int i2 = 0; i2 < 16; i2++) {
        const int pl = lane / 16 + 4 * i2;
        const uint32_t vw[4] = {vf[i2].x, vf[i2].y, vf[i2].z, vf[i2].w};
        float v[8];
#pragma unroll
        for (int e = 0; e < 4; e++) {
          v[2 * e] = lo16<DT_BF16>(vw[e]);
          v[2 * e + 1] = hi16<DT_BF16>(vw[e]);
        }
#pragma unroll
        for (int rr = 0; rr < 16; rr++) {
          const float p = pw[rr * 64 + pl];
#pragma unroll
          for (int e = 0; e < 8; e++) o_acc[rr][e] = fmaf(p, v[e], o_acc[rr][e]);
        }
      }
      __builtin_amdgcn_s_waitcnt(0xc07f);
      __builtin_amdgcn_wave_barrier();
    };
    // cached positions [c0, c1) of this split
    for (int blk = 0; blk < nblk; blk++) {
      const int p0 = c0 + blk * 64, plast = c1 - 1;
      uint4 kf[4][4], vf[16];
#pragma unroll
      for (int jb = 0; jb < 4; jb++) {
        const int p = min(p0 + 16 * jb + lane % 16, plast);
        const int pg = gptr(m.kv_indices)[pb + p / kPage];
        const uint16_t* src = op.k_cache + ((size_t)pg * kPage + p % kPage) * tok_stride + (size_t)h * D + (lane / 16) * 8;
#pragma unroll
        for (int q = 0; q < 4; q++) kf[jb][q] = ldg16(src + 32 * q);
      }
#pragma unroll
      for (int i2 = 0; i2 < 16; i2++) {
        const int p = min(p0 + lane / 16 + 4 * i2, plast);
        const int pg = gptr(m.kv_indices)[pb + p / kPage];
        vf[i2] = ldg16(op.v_cache + ((size_t)pg * kPage + p % kPage) * tok_stride + (size_t)h * D + (lane % 16) * 8);
      }
      const int npos = c1 - p0 < 64 ? c1 - p0 : 64;
      block(kf, vf, npos, false, 0);
    }
    // the new tokens (last split), 64 at a time, from LDS
    if (last) {
      for (int n0 = 0; n0 < nt; n0 += 64) {
        uint4 kf[4][4], vf[16];
        const int ilast = nt - 1;
#pragma unroll
        for (int jb = 0; jb < 4; jb++) {
          const int i = min(n0 + 16 * jb + lane % 16, ilast);
#pragma unroll
          for (int q = 0; q < 4; q++)
            kf[jb][q] = *reinterpret_cast<const uint4*>(knew + (size_t)i * D + 32 * q + (lane / 16) * 8);
        }
#pragma unroll
        for (int i2 = 0; i2 < 16; i2++) {
          const int i = min(n0 + lane / 16 + 4 * i2, ilast);
          vf[i2] = *reinterpret_cast<const uint4*>(vnew + (size_t)i * D + (lane % 16) * 8);
        }
        // causal: new position n0 + pl is visible to token tj iff n0 + pl <= tj
        block(kf, vf, nt - n0 < 64 ? nt - n0 : 64, true, n0);
      }
    }
    // rows' (o, m, l) into the split record: sum o over the 4 lane groups
#pragma unroll
    for (int rr = 0; rr < 16; rr++)
#pragma unroll
      for (int e = 0; e < 8; e++) {
        o_acc[rr][e] = add_xor32(add_xor16(o_acc[rr][e]));
      }
    if (lane < 16) {
#pragma unroll
      for (int rr = 0; rr < 16; rr++) {
        const int row = 16 * rb + rr;
        if (row < R) {
          float* dst = rec + (size_t)row * (D + 2) + lane * 8;
          st_agent4(dst, make_float4(o_acc[rr][0], o_acc[rr][1], o_acc[rr][2], o_acc[rr][3]));
          st_agent4(dst + 4, make_float4(o_acc[rr][4], o_acc[rr][5], o_acc[rr][6], o_acc[rr][7]));
        }
      }
    }
    if ((lane % 16) == 0) {
#pragma unroll
      for (int i = 0; i < 4; i++) {
        const int row = 16 * rb + 4 * (lane / 16) + i;
        if (row < R) {
          st_agent(rec + (size_t)row * (D + 2) + D, m_i[i]);
          st_agent(rec + (size_t)row * (D + 2) + D + 1, l_i[i]);
        }
      }
    }
  }
  // the last split task to arrive merges every row's S records
  if (arrive_last(&a.tickets[op.ticket_base + r * op.num_kv_heads + h], S)) {
    for (int idx = tix(); idx < R * (D / 4); idx += PK_THREADS) {
      const int rr = idx / (D / 4), d4 = (idx % (D / 4)) * 4;
      float M = -INFINITY, L = 0.f;
      float4 O = make_float4(0.f, 0.f, 0.f, 0.f);
      // records in split order, 4 splits' loads in flight per round trip
      for (int s0 = 0; s0 < S; s0 += 4) {
        float msv[4], lsv[4];
        float4 osv[4];
#pragma unroll
        for (int j = 0; j < 4; j++) {
          const float* rc = rec_base + (size_t)(s0 + j) * rec_floats + (size_t)rr * (D + 2);
          const bool ok = s0 + j < S;
          msv[j] = ok ? ld_agent(rc + D) : -INFINITY;
          lsv[j] = ok ? ld_agent(rc + D + 1) : 0.f;
          osv[j] = ok ? ld_agent4(rc + d4) : make_float4(0.f, 0.f, 0.f, 0.f);
        }
#pragma unroll
        for (int j = 0; j < 4; j++) {
          const float ms = msv[j];
          if (ms == -INFINITY) continue;
          const float mn = fmaxf(M, ms);
          const float fa = M == -INFINITY ? 0.f : exp2f(M - mn), fb = exp2f(ms - mn);
          L = L * fa + lsv[j] * fb;
          O.x = O.x * fa + osv[j].x * fb; O.y = O.y * fa + osv[j].y * fb;
          O.z = O.z * fa + osv[j].z * fb; O.w = O.w * fa + osv[j].w * fb;
          M = mn;
        }
      }
      const float inv = L > 0.f ? 1.f / L : 0.f;
      const int jt = rr / G, g = rr % G;
      const size_t oe = (size_t)(t0 + jt) * op.out_ld + (size_t)(h * G + g) * D + d4;
      const uint32_t lo = pack2<DT_BF16>(O.x * inv, O.y * inv), hi = pack2<DT_BF16>(O.z * inv, O.w * inv);
      __hip_atomic_store(gptr(reinterpret_cast<uint64_t*>(op.out + oe)), (uint64_t)lo | ((uint64_t)hi << 32),
                         __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
  }
  signal_event(a, t);
}

// ------------------------------------------------------------ batch manager
// Offline-mode prepare_next_batch (persistent_kernel.cuh:169-322), run by one
// thread; integer logic identical to the CPU restatement in the oracle.
__device__ __forceinline__ void task_prepare(const KernelArgs& a, const TaskDesc& t, int task_id, Shared& sm) {
  if (!wait_event(a, t, task_id, sm)) return;
  if (tix() == 0 && a.meta.online) {
    // online mode (persistent_kernel.cuh:325-351): one request; the host
    // feeds how many tokens this step produced
    const BatchMeta& s = a.meta;
    const int step = gptr(s.step)[0];
    gptr(s.step)[0] = step + gptr(s.num_new_tokens)[0];
    gptr(s.status)[1] = !(step + 2 >= s.max_seq_len || gptr(s.tokens)[step + 1] == s.eos_token_id);
  } else if (tix() == 0) {
    const BatchMeta& s = a.meta;
    const int MR = s.max_requests, MT = s.max_tokens, MP = s.max_pages, PS = s.page_size, MSL = s.max_seq_len;
    int head = *s.page_queue_head, tail = *s.page_queue_tail;
    for (int i = 0; i < MR; i++) {
      int rid = gptr(s.request_ids)[i];
      if (rid == -1) continue;
      int step = gptr(s.step)[rid], qo = gptr(s.qo_indptr)[i], nt = gptr(s.qo_indptr)[i + 1] - qo, plen = gptr(s.prompt_lengths)[rid];
      for (int j = 0; j < nt; j++)
        if (step + j + 1 >= plen && step + j + 1 < MSL)
          gptr(s.tokens)[(size_t)rid * MSL + step + j + 1] =
              (int64_t)__hip_atomic_load(gptr(reinterpret_cast<uint64_t*>(s.output_tokens + qo + j)), __ATOMIC_RELAXED,
                                         __HIP_MEMORY_SCOPE_AGENT);
      gptr(s.step)[rid] = step + nt;
      if ((step + nt + 1 >= MSL) ||
          ((gptr(s.tokens)[(size_t)rid * MSL + step + nt] == s.eos_token_id) && (step + nt >= plen))) {
        gptr(s.request_ids)[i] = -1;
        int kp = gptr(s.kv_indptr)[i], npg = gptr(s.kv_indptr)[i + 1] - kp;
        for (int j = 0; j < npg; j++) { gptr(s.page_queue)[tail % MP] = gptr(s.kv_indices)[kp + j]; tail++; }
      }
    }
    // the page table is rebuilt in place: requests keep their old pages from
    // a snapshot (device memory of max_pages ids owned by the handle)
    int* snap = s.page_snap;
    const int all = gptr(s.kv_indptr)[MR];
    for (int i = 0; i < all && i < MP; i++) snap[i] = gptr(s.kv_indices)[i];
    int nreq = 0, ntok = 0, npg = 0;
    for (int i = 0; i < MR; i++) {
      int rid = gptr(s.request_ids)[i];
      if (rid == -1) continue;
      int kp = gptr(s.kv_indptr)[i], nold = gptr(s.kv_indptr)[i + 1] - kp;
      gptr(s.request_ids)[nreq] = rid;
      gptr(s.qo_indptr)[nreq] = ntok;
      gptr(s.kv_indptr)[nreq] = npg;
      int step = gptr(s.step)[rid];
      int nnew = gptr(s.prompt_lengths)[rid] - step;
      nnew = nnew > 0 ? (nnew < MT - ntok ? nnew : MT - ntok) : (1 < MT - ntok ? 1 : MT - ntok);
      for (int j = 0; j < nnew; j++) gptr(s.input_tokens)[ntok + j] = gptr(s.tokens)[(size_t)rid * MSL + step + j];
      int nnp = (step + nnew + PS - 1) / PS;
      gptr(s.last_page_len)[nreq] = (step + nnew) % PS;
      for (int j = 0; j < nold; j++) gptr(s.kv_indices)[npg + j] = snap[kp + j];
      for (int j = nold; j < nnp; j++) { gptr(s.kv_indices)[npg + j] = gptr(s.page_queue)[head % MP]; head++; }
      npg += nnp;
      ntok += nnew;
      nreq++;
    }
    while (nreq < MR && ntok < MT) {
      int nid = *s.next_request_id;
      if (nid >= s.total_requests) break;
      gptr(s.request_ids)[nreq] = nid;
      gptr(s.qo_indptr)[nreq] = ntok;
      gptr(s.kv_indptr)[nreq] = npg;
      int nnew = gptr(s.prompt_lengths)[nid] < MT - ntok ? gptr(s.prompt_lengths)[nid] : MT - ntok;
      for (int j = 0; j < nnew; j++) gptr(s.input_tokens)[ntok + j] = gptr(s.tokens)[(size_t)nid * MSL + j];
      int nnp = (nnew + PS - 1) / PS;
      gptr(s.last_page_len)[nreq] = nnew % PS;
      for (int j = 0; j < nnp; j++) { gptr(s.kv_indices)[npg + j] = gptr(s.page_queue)[head % MP]; head++; }
      ntok += nnew;
      npg += nnp;
      nreq++;
      *s.next_request_id = nid + 1;
    }
    for (int i = nreq; i < MR; i++) gptr(s.request_ids)[i] = -1;
    for (int i = nreq; i <= MR; i++) { gptr(s.qo_indptr)[i] = ntok; gptr(s.kv_indptr)[i] = npg; }
    *s.page_queue_head = head;
    *s.page_queue_tail = tail;
    gptr(s.status)[1] = ntok != 0;
  }
  signal_event(a, t);
}

// Attention tasks among descriptor slots [0, n) of the first descriptor
// chunk: their request geometry and the page ids of their first blocks from
// the batch metadata (one thread per slot; at most kPreMax tasks, the rest
// read the metadata themselves).
__device__ __forceinline__ void fill_pre(const KernelArgs& a, int n, Shared& sm) {
  const int k = tix();
  if (k == 0) sm.pre_n = 0;
  __syncthreads();
  if (k < n) {
    int idx = kPreNone;
    const TaskDesc& t = sm.tq[k];
    OpRef op = op_of(a, t.op);
    if (op.type == TASK_ATTENTION) {
      const int e = atomicAdd(&sm.pre_n, 1);
      if (e < kPreMax) {
        idx = e;
        const BatchMeta& m = a.meta;
        const AttnGeom g = attn_geom(m, op, t.i0, t.i2);
        AttnPre& P = sm.pre[e];
        P.t0 = g.t0; P.nt = g.nt; P.pb = g.pb; P.np = g.np; P.base = g.base; P.c0 = g.c0; P.c1 = g.c1;
        for (int w = 0; w < 7; w++) {
          const int p0 = g.c0 + w * 64;
          int idA = 0, idB = 0;
          if (g.nt > 0 && p0 < g.c1) {
            const int pg0 = p0 / kPage;
            idA = gptr(m.kv_indices)[g.pb + pg0];
            idB = pg0 + 1 < g.np ? gptr(m.kv_indices)[g.pb + pg0 + 1] : idA;
          }
          P.id[2 * w] = idA;
          P.id[2 * w + 1] = idB;
        }
        for (int i = 0; i < 4; i++) P.pg_tok[i] = i < g.nt ? gptr(m.kv_indices)[g.pb + (g.base + i) / kPage] : 0;
      }
    }
    sm.pre_of[k] = (uint8_t)idx;
  }
  __syncthreads();
}

// ------------------------------------------------------------ kernel
// ------------------------------------------------------------ task entry points
// Each task type is its own function: the worker loop calls it with the
// descriptor's LDS slot; the descriptor is copied into scalar registers here.
__device__ __forceinline__ TaskDesc task_at(int slot) {
  TaskDesc t;
  const uint32_t* src = reinterpret_cast<const uint32_t*>(&g_sm.tq[__builtin_amdgcn_readfirstlane(slot)]);
  uint32_t* dst = reinterpret_cast<uint32_t*>(&t);
#pragma unroll
  for (int e = 0; e < (int)(sizeof(TaskDesc) / 4); e++) dst[e] = __builtin_amdgcn_readfirstlane(src[e]);
  return t;
}

template <int TM, int EPI, bool PK>
__device__ __forceinline__ void run_gemv(int slot, int tid) {
  const TaskDesc t = task_at(slot);
  task_gemv<TM, EPI, PK>(g_sm.args, t, __builtin_amdgcn_readfirstlane(tid), g_sm);
}
// batches of 9..16 tokens (chunked prefill): out of line, so the decode
// paths keep their code layout
template <int EPI, bool PK>
__device__ __attribute__((noinline)) void run_gemv16(int slot, int tid) {
  const TaskDesc t = task_at(slot);
  task_gemv<16, EPI, PK>(g_sm.args, t, __builtin_amdgcn_readfirstlane(tid), g_sm);
}
template <int RMAX>
__device__ __forceinline__ void run_attention(int slot, int tid) {
  const TaskDesc t = task_at(slot);
  task_attention_body<RMAX>(g_sm.args, t, __builtin_amdgcn_readfirstlane(tid), slot, g_sm);
}
// the multi-token variant (rare on the decode path, heavy register use) stays
// out of line so that it cannot push the hot paths into spilling
__device__ __attribute__((noinline)) void run_attention_large(int slot, int tid) {
  const TaskDesc t = task_at(slot);
  task_attention_body<16>(g_sm.args, t, __builtin_amdgcn_readfirstlane(tid), slot, g_sm);
}
// prefill / extend rows (nt * G > 16): out of line for the same reason
__device__ __attribute__((noinline)) void run_attention_mt(int slot, int tid) {
  const TaskDesc t = task_at(slot);
  task_attention_mt(g_sm.args, t, __builtin_amdgcn_readfirstlane(tid), g_sm);
}
__device__ __forceinline__ void run_embed(int slot, int tid) {
  const TaskDesc t = task_at(slot);
  task_embed(g_sm.args, t, __builtin_amdgcn_readfirstlane(tid), g_sm);
}
__device__ __forceinline__ void run_prepare(int slot, int tid) {
  const TaskDesc t = task_at(slot);
  task_prepare(g_sm.args, t, __builtin_amdgcn_readfirstlane(tid), g_sm);
}

// Grid barrier between task-graph passes.  Every wave first releases its
// stores at agent scope (the KV appends, the batch metadata prepare_batch
// rewrote and the profile words are plain stores that may sit in this XCD's
// L2); one arrival per worker; the arrival count says which barrier this is
// (arrivals grow by num_workers per barrier), so the counter needs no epoch.
// After the barrier every wave invalidates its non-coherent cache lines, so
// the next pass reads the other workers' writes.  Returns false when the
// watchdog fired or the launch aborted.
__device__ __attribute__((noinline)) bool grid_barrier(const KernelArgs& a, Shared& sm) {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "agent");
  __syncthreads();
  if (threadIdx.x == 0) {
    int ok = 1;
    const uint32_t n = (uint32_t)a.num_workers;
    const uint32_t arr = __hip_atomic_fetch_add(gptr(a.grid_bar), 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    const uint32_t target = (arr / n + 1) * n;
    long long spins = 0;
    for (;;) {
      const uint32_t v = __hip_atomic_load(gptr(a.grid_bar), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      if ((int32_t)(v - target) >= 0) break;
      if ((spins & 255) == 255 && aborted(a)) { ok = 0; break; }
      if (++spins > a.spin_limit) {
        __hip_atomic_store(gptr(a.meta.status + 2), -2, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        __hip_atomic_store(gptr(a.meta.status), 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        ok = 0;
        break;
      }
      __builtin_amdgcn_s_sleep(2);
    }
    sm.flag = ok;
  }
  __syncthreads();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
  return sm.flag != 0;
}

// Linear task of a graph whose batches hold up to MT tokens (1, 8 or 16):
// one token-tile width per kernel instance, so each instance carries only
// its own GEMV code (the worker loop is sensitive to its code footprint).
template <int MT, bool PK, int EPI>
__device__ __forceinline__ void run_linear(int slot, int tid) {
  if constexpr (MT == 16) run_gemv16<EPI, PK>(slot, tid);
  else run_gemv<MT, EPI, PK>(slot, tid);
}

// After an early stop: every event counter advanced by num_triggers x the
// passes that did not run (worker w takes events w, w + workers, ...).
__device__ __attribute__((noinline)) void fast_forward(const KernelArgs& a, int w, uint32_t skip) {
  for (int e = w * PK_THREADS + tix(); e < a.num_events; e += a.num_workers * PK_THREADS)
    __hip_atomic_fetch_add(gptr(&a.events[e]), gptr(a.event_triggers)[e] * skip, __ATOMIC_RELAXED,
                           __HIP_MEMORY_SCOPE_AGENT);
}

// MT: token-tile width (1, 8, 16); PK: batch > 1 linear tasks read weights
// packed in stream order (yr_pk_pack_weights).  One instance per pair, so
// each carries only its own linear-task code.
template <int MT, bool PK>
__global__ __launch_bounds__(PK_THREADS, 1) void pk_worker_kernel(KernelArgs a) {
  Shared& sm = g_sm;
  const int w = blockIdx.x;
  const int q0 = gptr(a.queue_offsets)[w], q1 = gptr(a.queue_offsets)[w + 1];
  // this worker's task descriptors move to LDS, 256 at a time
  auto load_descs = [&](int first) __attribute__((always_inline)) {
    const int n = q1 - first < 256 ? q1 - first : 256;
    const int words = (int)(sizeof(TaskDesc) / 4);
    for (int i = tix(); i < n * words; i += PK_THREADS) {
      int k = i / words, e = i % words;
      const int id = gptr(a.queue)[first + k];
      reinterpret_cast<uint32_t*>(&sm.tq[k])[e] = gptr(reinterpret_cast<const uint32_t*>(&a.tasks[id]))[e];
      if (e == 0) sm.tq_id[k] = id;
    }
  };
  load_descs(q0);
  int it = 0;
  for (;;) {  // task-graph passes (epochs a.epoch + it)
  __syncthreads();
  fill_pre(a, q1 - q0 < 256 ? q1 - q0 : 256, sm);
  if (threadIdx.x == 0) {
    sm.args = a;
    sm.args.epoch = a.epoch + (uint32_t)it;
    sm.flag = 1;
    sm.last_op = -1;  // staged activations belong to the previous pass
    sm.last_T = 0;
    sm.norm_rows = 0;
    sm.coop_stage = 0;
  }
  __syncthreads();
  for (int q = q0; q < q1; q++) {
    if (q > q0 && (q - q0) % 256 == 0) {
      __syncthreads();
      load_descs(q);
      // (later descriptor chunks: attention tasks read their metadata)
      for (int i = tix(); i < 256; i += PK_THREADS) sm.pre_of[i] = kPreNone;
      __syncthreads();
    }
    const int slot = (q - q0) % 256;
    // (task ids come from LDS: a global read here would put a dependent
    // memory round trip at the start of every task)
    const int tid = __builtin_amdgcn_readfirstlane(sm.tq_id[slot]);
    OpRef op = op_of(a, sm.tq[slot].op);
    if (a.profile && threadIdx.x == 0) {
      gptr(a.profile)[(size_t)tid * 8] = now_10ns();
      gptr(a.profile)[(size_t)tid * 8 + 3] = (uint64_t)w;
    }
    const int type = op.type;
    const bool gemv = type == TASK_LINEAR || type == TASK_RMSNORM_LINEAR || type == TASK_RMSNORM_LINEAR_SILU ||
                      type == TASK_RMSNORM_LINEAR_ARGMAX;
    if (!gemv && threadIdx.x == 0) sm.last_op = -1;  // attention / embed / batch tasks reuse xs
    switch (type) {
      case TASK_EMBED: run_embed(slot, tid); break;
      case TASK_LINEAR:
        run_linear<MT, PK, EPI_LIN>(slot, tid);
        break;
      case TASK_RMSNORM_LINEAR:
        run_linear<MT, PK, EPI_NORM>(slot, tid);
        break;
      case TASK_RMSNORM_LINEAR_SILU:
        run_linear<MT, PK, EPI_SILU>(slot, tid);
        break;
      case TASK_RMSNORM_LINEAR_ARGMAX:
        run_linear<MT, PK, EPI_ARGMAX>(slot, tid);
        break;
      case TASK_ATTENTION: {
        // query rows per kv head: nt * G (one MFMA row block of 4 or 16)
        const int G = op.num_q_heads / op.num_kv_heads;
        bool small = op.max_tokens * G <= 4;
        if (!small) {
          const int r = sm.tq[slot].i0;
          small = (gptr(a.meta.qo_indptr)[r + 1] - gptr(a.meta.qo_indptr)[r]) * G <= 4;
        }
        if (small) {
          run_attention<4>(slot, tid);
        } else {
          const int r = sm.tq[slot].i0;
          const int nt = gptr(a.meta.qo_indptr)[r + 1] - gptr(a.meta.qo_indptr)[r];
          if (nt * G > 16) run_attention_mt(slot, tid); else run_attention_large(slot, tid);
        }
        break;
      }
      case TASK_PREPARE_BATCH: run_prepare(slot, tid); break;
      default: break;
    }
    // GEMV tasks need no trailing barrier: the next task's first LDS access
    // comes after its own [X] barrier, which the sync wave reaches only after
    // publishing this task, so the compute waves run ahead and put the next
    // task's weights in flight meanwhile
    if (!gemv) lds_sync();
    if (a.profile && threadIdx.x == 0) gptr(a.profile)[(size_t)tid * 8 + 2] = now_10ns();
    if (!sm.flag) return;  // a dependency never arrived: leave the queue
  }
  if (it + 1 >= a.max_iterations) break;
  // every worker finished pass `it` (prepare_batch included) before any
  // starts the next one: the next pass re-reads the batch metadata
  // (the LDS copy of the arguments: passing the kernel argument itself by
  // reference to an out-of-line function would put it in scratch memory, and
  // every later field read would become a memory round trip)
  if (!grid_barrier(sm.args, sm)) return;
  if (threadIdx.x == 0)
    sm.flag = !a.stop_when_empty ||
              __hip_atomic_load(gptr(a.meta.status + 1), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) != 0;
  __syncthreads();
  if (!sm.flag) {
    // Early stop: bring every event to where max_iterations passes would
    // have left it, so the next launch (epoch a.epoch + max_iterations, as
    // the host counts) waits for the right values.  Nobody waits on an
    // event in this launch any more (all workers passed the barrier).
    fast_forward(sm.args, w, (uint32_t)(a.max_iterations - 1 - it));
    break;
  }
  it++;
  if (q1 - q0 > 256) load_descs(q0);  // the queue's first chunk again
  }
  if (w == 0 && threadIdx.x == 0) gptr(a.iterations_run)[0] = it + 1;
}

// Batch state initialisation (persistent_kernel.cuh:107-132).
__global__ void pk_init_batch_kernel(BatchMeta s) {
  if (threadIdx.x == 0 && blockIdx.x == 0) {
    for (int i = 0; i < s.total_requests; i++) gptr(s.step)[i] = 0;
    *s.next_request_id = 0;
    for (int i = 0; i < s.max_requests; i++) gptr(s.request_ids)[i] = -1;
    for (int i = 0; i < s.max_requests + 1; i++) { gptr(s.qo_indptr)[i] = 0; gptr(s.kv_indptr)[i] = 0; }
    *s.page_queue_head = 0;
    *s.page_queue_tail = s.max_pages;
    for (int i = 0; i < s.max_pages; i++) gptr(s.page_queue)[i] = i;
  }
}

// One linear task's weights in the order its batch > 1 stream reads them:
// unit p = (block kb, 16-row tile, 32-column chunk c), 64 lanes x 16 bytes,
// lane l = row 16 tile + l % 16 (clamped to the last row), columns
// kb KB + 32 c + 8 (l / 16) .. + 8 -- the MFMA A fragment task_gemv loads.
struct PackJob {
  const uint16_t* w0;
  const uint16_t* w1;
  uint16_t* dst;
  unsigned long long unit0;  // first global unit of this task's stream
  int seg, RT, K, KB, NT, UPR;
};
// Every task's stream in one launch: global unit u belongs to the job whose
// [unit0, next unit0) holds it (binary search over the sorted job table).
__global__ void pk_pack_kernel(const PackJob* jobs, int njobs, unsigned long long units) {
  for (unsigned long long i = (unsigned long long)blockIdx.x * blockDim.x + threadIdx.x; i < units * kWave;
       i += (unsigned long long)gridDim.x * blockDim.x) {
    const unsigned long long u = i / kWave;
    const int l = (int)(i % kWave);
    int lo = 0, hi = njobs - 1;
    while (lo < hi) {
      const int mid = (lo + hi + 1) >> 1;
      if (jobs[mid].unit0 <= u) lo = mid; else hi = mid - 1;
    }
    const PackJob& j = jobs[lo];
    const size_t p = (size_t)(u - j.unit0);
    const int kb = (int)(p / ((size_t)j.NT * j.UPR)), rem = (int)(p % ((size_t)j.NT * j.UPR));
    const int tile = rem / j.UPR, c = rem % j.UPR;
    const int r = min(tile * 16 + l % 16, j.RT - 1);
    const uint16_t* src = (r < j.seg ? j.w0 + (size_t)r * j.K : j.w1 + (size_t)(r - j.seg) * j.K) +
                          (size_t)kb * j.KB + c * 32 + (l / 16) * 8;
    *reinterpret_cast<uint4*>(j.dst + p * 512 + l * 8) = *reinterpret_cast<const uint4*>(src);
  }
}

__global__ void pk_fill_u32_kernel(uint32_t* p, size_t n, uint32_t v) {
  for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (size_t)gridDim.x * blockDim.x) p[i] = v;
}

// ------------------------------------------------------------ host handle
// Passes one launch may run, and the epoch at which the host re-bases the
// counters: link tags hold the epoch in 32 - kLinkOpBits = 22 bits, and a
// wait compares counters up to num_triggers * epoch (< 2^31 for <= 512
// triggers) with a wrap-safe difference.
constexpr int kMaxIterations = 1 << 20;
constexpr uint32_t kEpochRebase = 1u << 21;

struct Handle {
  int device = 0;
  int num_workers = 0;
  size_t n_ops = 0, n_tasks = 0, n_events = 0, n_tickets = 0;
  OpDesc* d_ops = nullptr;
  TaskDesc* d_tasks = nullptr;
  int* d_qoff = nullptr;
  int* d_queue = nullptr;
  uint32_t* d_events = nullptr;     // [n_events] counters, then the grid-barrier counter
  uint32_t* d_triggers = nullptr;   // [n_events] num_triggers
  int* d_iters = nullptr;           // [1] passes the last launch ran
  uint32_t* d_tickets = nullptr;
  float* d_scratch = nullptr;
  int* d_status = nullptr;
  int* d_owned_meta = nullptr;  // request_ids, next_request_id, page_queue, head, tail, page snapshot
  BatchMeta meta;
  uint32_t epoch = 0;  // epoch of the last pass the device may have run
  long long spin_limit = 1ll << 26;
  bool has_prepare = false;
  const void* kfn = nullptr;         // pk_worker_kernel<1 / 8 / 16, false>
  const void* kfn_packed = nullptr;  // pk_worker_kernel<8 / 16, true> (weights packed)
  bool cooperative = true;
  uint64_t* profile = nullptr;
  std::vector<std::pair<uint64_t, uint64_t>> link_buffers;  // tags restart with the epochs: cleared then
  size_t scratch_words = 0;                                  // d_scratch, in 32-bit words
  int tm = 1;                                                // token-tile width of the kernel instance
  std::vector<TaskDesc> tasks;                               // host copy (weight pointers as built)
  std::vector<OpDesc> ops;
  uint16_t* d_packed = nullptr;                              // packed linear weights (yr_pk_pack_weights)
};

// Zero every word that carries an epoch tag: the link tensors and the
// scratch area (the attention split records), since the tags restart with
// the epochs.  A record slot that some pass left behind (a request mix that
// no longer uses it) would otherwise match a restarted epoch's tag.
static int clear_tagged(Handle* h, hipStream_t st) {
  for (auto& lb : h->link_buffers) {
    hipLaunchKernelGGL(pk_fill_u32_kernel, dim3(256), dim3(256), 0, st, reinterpret_cast<uint32_t*>(lb.first),
                       (size_t)(lb.second / 4), 0u);
    YR_CHECK_LAUNCH("pk_fill_u32_kernel (link tensors)");
  }
  hipLaunchKernelGGL(pk_fill_u32_kernel, dim3(256), dim3(256), 0, st, reinterpret_cast<uint32_t*>(h->d_scratch),
                     h->scratch_words, 0u);
  YR_CHECK_LAUNCH("pk_fill_u32_kernel (scratch)");
  return YR_OK;
}

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
  // the kernel instance for the graph's token-tile width
  const int mt = g->cfg.max_tokens;
  const void* kfn = mt <= 1 ? reinterpret_cast<const void*>(pk_worker_kernel<1, false>)
                    : mt <= 8 ? reinterpret_cast<const void*>(pk_worker_kernel<8, false>)
                              : reinterpret_cast<const void*>(pk_worker_kernel<16, false>);
  const void* kfn_packed = mt <= 1 ? nullptr
                           : mt <= 8 ? reinterpret_cast<const void*>(pk_worker_kernel<8, true>)
                                     : reinterpret_cast<const void*>(pk_worker_kernel<16, true>);
  int occ = 0;
  if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&occ, kfn, PK_THREADS, 0) != hipSuccess)
    return fail(YR_E_HIP, "yr_pk_create: occupancy query failed");
  if (kfn_packed) {
    int occ2 = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&occ2, kfn_packed, PK_THREADS, 0) != hipSuccess)
      return fail(YR_E_HIP, "yr_pk_create: occupancy query failed");
    occ = std::min(occ, occ2);
  }
  if (g->num_workers > occ * prop.multiProcessorCount)
    return fail(YR_E_INVALID, "yr_pk_create: %d workers cannot be co-resident (%d CUs x %d)", g->num_workers,
                prop.multiProcessorCount, occ);
  Handle* h = new Handle();
  h->kfn = kfn;
  h->kfn_packed = kfn_packed;
  h->device = dev;
  h->num_workers = g->num_workers;
  h->n_ops = g->ops.size();
  h->n_tasks = g->tasks.size();
  h->n_events = g->events.size();
  h->link_buffers = g->link_buffers;
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
  YRA(h->d_events, sizeof(uint32_t) * (h->n_events + 1));
  YRA(h->d_triggers, sizeof(uint32_t) * h->n_events);
  YRA(h->d_iters, sizeof(int) * 4);
  YRA(h->d_tickets, sizeof(uint32_t) * (g->num_tickets + 1));
  YRA(h->d_scratch, sizeof(float) * (g->scratch_floats + 4));
  h->scratch_words = g->scratch_floats + 4;
  h->tm = mt <= 1 ? 1 : mt <= 8 ? 8 : 16;
  h->tasks = g->tasks;
  h->ops = g->ops;
  h->n_tickets = g->num_tickets;
  YRA(h->d_status, sizeof(int) * 4);
  const int MR = g->cfg.max_requests, MP = g->cfg.max_pages;
  YRA(h->d_owned_meta, sizeof(int) * (MR + 1 + MP + 2 + MP));
#undef YRA
  if (rc == YR_OK) rc = hip_ok(hipMemcpy(h->d_ops, g->ops.data(), sizeof(OpDesc) * h->n_ops, hipMemcpyHostToDevice), "copy ops");
  if (rc == YR_OK) rc = hip_ok(hipMemcpy(h->d_tasks, g->tasks.data(), sizeof(TaskDesc) * h->n_tasks, hipMemcpyHostToDevice), "copy tasks");
  if (rc == YR_OK) rc = hip_ok(hipMemcpy(h->d_qoff, qoff.data(), sizeof(int) * qoff.size(), hipMemcpyHostToDevice), "copy queues");
  if (rc == YR_OK && queue.size()) rc = hip_ok(hipMemcpy(h->d_queue, queue.data(), sizeof(int) * queue.size(), hipMemcpyHostToDevice), "copy queues");
  if (rc == YR_OK) rc = hip_ok(hipMemset(h->d_events, 0, sizeof(uint32_t) * (h->n_events + 1)), "clear events");
  if (rc == YR_OK) rc = hip_ok(hipMemset(h->d_iters, 0, sizeof(int) * 4), "clear iterations");
  if (rc == YR_OK && h->n_events) {
    std::vector<uint32_t> trig(h->n_events);
    for (size_t e = 0; e < h->n_events; e++) trig[e] = (uint32_t)g->events[e].num_triggers;
    rc = hip_ok(hipMemcpy(h->d_triggers, trig.data(), sizeof(uint32_t) * h->n_events, hipMemcpyHostToDevice),
                "copy event triggers");
  }
  for (const OpDesc& o : g->ops)
    if (o.type == TASK_PREPARE_BATCH) h->has_prepare = true;
  if (rc == YR_OK) rc = hip_ok(hipMemset(h->d_tickets, 0, sizeof(uint32_t) * (g->num_tickets + 1)), "clear tickets");
  if (rc == YR_OK) rc = hip_ok(hipMemset(h->d_status, 0, sizeof(int) * 4), "clear status");
  if (rc == YR_OK) rc = hip_ok(hipMemset(h->d_scratch, 0, sizeof(float) * h->scratch_words), "clear scratch");
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
  m.page_snap = h->d_owned_meta + MR + 3 + MP;
  m.status = h->d_status;
  m.max_requests = MR;
  m.max_tokens = g->cfg.max_tokens;
  m.max_pages = MP;
  m.page_size = g->cfg.page_size;
  m.max_seq_len = g->cfg.max_seq_len;
  m.total_requests = g->cfg.total_requests;
  m.eos_token_id = g->cfg.eos_token_id;
  m.online = g->cfg.online;
  if (m.online && h->has_prepare && (!m.num_new_tokens || !m.step || !m.tokens)) {
    yr_pk_destroy(reinterpret_cast<yr_pk_handle*>(h));
    return fail(YR_E_INVALID, "yr_pk_create: online mode needs step, tokens and num_new_tokens");
  }
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

int yr_pk_launch(yr_pk_handle* hp, void* stream, int max_iterations) {
  Handle* h = reinterpret_cast<Handle*>(hp);
  if (!h) return fail(YR_E_INVALID, "yr_pk_launch: null handle");
  if (max_iterations < 0 || max_iterations > kMaxIterations)
    return fail(YR_E_INVALID, "yr_pk_launch: max_iterations %d outside [0, %d]", max_iterations, kMaxIterations);
  if (max_iterations == 0) {
    // until the batch is empty: only a graph with a prepare_batch task knows when
    if (!h->has_prepare)
      return fail(YR_E_INVALID, "yr_pk_launch: max_iterations 0 (run to completion) needs a prepare_batch task");
    max_iterations = kMaxIterations;
  }
  hipStream_t st = (hipStream_t)stream;
  // counters are monotonic; re-base them well before the link tags
  // (epoch << kLinkOpBits in 32 bits) or the counters wrap
  if (h->epoch + (uint32_t)max_iterations >= kEpochRebase) {
    hipLaunchKernelGGL(pk_fill_u32_kernel, dim3(64), dim3(256), 0, st, h->d_events, h->n_events + 1, 0u);
    YR_CHECK_LAUNCH("pk_fill_u32_kernel");
    int rc = clear_tagged(h, st);
    if (rc != YR_OK) return rc;
    h->epoch = 0;
  }
  KernelArgs a;
  a.ops = h->d_ops;
  a.tasks = h->d_tasks;
  a.queue_offsets = h->d_qoff;
  a.queue = h->d_queue;
  a.events = h->d_events;
  a.tickets = h->d_tickets;
  a.scratch = h->d_scratch;
  a.meta = h->meta;
  a.epoch = h->epoch + 1;
  a.num_workers = h->num_workers;
  a.spin_limit = h->spin_limit;
  a.profile = h->profile;
  a.max_iterations = max_iterations;
  a.stop_when_empty = h->has_prepare ? 1 : 0;
  a.grid_bar = h->d_events + h->n_events;
  a.event_triggers = h->d_triggers;
  a.num_events = (int)h->n_events;
  a.iterations_run = h->d_iters;
  // the device ends at epoch + max_iterations whether or not it stops early
  // (an early stop fast-forwards the counters)
  h->epoch += (uint32_t)max_iterations;
  void* args[] = {&a};
  const void* fn = h->d_packed ? h->kfn_packed : h->kfn;
  hipError_t e;
  if (h->cooperative)
    e = hipLaunchCooperativeKernel(fn, dim3(h->num_workers),
                                   dim3(PK_THREADS), args, 0, st);
  else
    e = hipLaunchKernel(fn, dim3(h->num_workers), dim3(PK_THREADS),
                        args, 0, st);
  if (e != hipSuccess) return check_hip(e, "launch of pk_worker_kernel");
  return YR_OK;
}

int yr_pk_iterations(yr_pk_handle* hp, int* iterations) {
  Handle* h = reinterpret_cast<Handle*>(hp);
  if (!h || !iterations) return fail(YR_E_INVALID, "yr_pk_iterations: bad arguments");
  hipError_t e = hipMemcpy(iterations, h->d_iters, sizeof(int), hipMemcpyDeviceToHost);
  if (e != hipSuccess) return check_hip(e, "yr_pk_iterations");
  return YR_OK;
}

int yr_pk_read_batch(yr_pk_handle* hp, int* out, size_t n) {
  Handle* h = reinterpret_cast<Handle*>(hp);
  if (!h || !out) return fail(YR_E_INVALID, "yr_pk_read_batch: bad arguments");
  const size_t need = (size_t)h->meta.max_requests + 3 + (size_t)h->meta.max_pages;
  if (n < need) return fail(YR_E_INVALID, "yr_pk_read_batch: needs %zu ints", need);
  hipError_t e = hipMemcpy(out, h->d_owned_meta, sizeof(int) * need, hipMemcpyDeviceToHost);
  if (e != hipSuccess) return check_hip(e, "yr_pk_read_batch");
  return YR_OK;
}

int yr_pk_set_launch_mode(yr_pk_handle* hp, int cooperative) {
  Handle* h = reinterpret_cast<Handle*>(hp);
  if (!h) return fail(YR_E_INVALID, "yr_pk_set_launch_mode: null handle");
  // co-residency of every worker was checked against the occupancy at create
  h->cooperative = cooperative != 0;
  return YR_OK;
}

int yr_pk_pack_weights(yr_pk_handle* hp, int enable, size_t* bytes) {
  Handle* h = reinterpret_cast<Handle*>(hp);
  if (!h) return fail(YR_E_INVALID, "yr_pk_pack_weights: null handle");
  if (bytes) *bytes = 0;
  std::vector<TaskDesc> tasks = h->tasks;
  if (h->d_packed) {
    (void)hipDeviceSynchronize();  // no launch may still read them
    (void)hipFree(h->d_packed);
    h->d_packed = nullptr;
  }
  if (enable && h->tm > 1) {
    // geometry of each batch > 1 linear task, as task_gemv derives it
    struct Job { size_t task, off, units; int RT, seg, K, KB, NT, UPR; };
    std::vector<Job> jobs;
    size_t total = 0;
    for (size_t i = 0; i < tasks.size(); i++) {
      const TaskDesc& t = tasks[i];
      const OpDesc& o = h->ops[t.op];
      const bool silu = o.type == TASK_RMSNORM_LINEAR_SILU;
      if (o.type != TASK_LINEAR && o.type != TASK_RMSNORM_LINEAR && !silu && o.type != TASK_RMSNORM_LINEAR_ARGMAX)
        continue;
      if (t.rows <= 0) continue;
      Job j;
      j.task = i;
      j.K = o.K;
      j.RT = silu ? 2 * t.rows : t.rows;
      j.seg = silu ? t.rows : t.split_row;
      const int NC = o.K >> 9, nkb = gemv_blocks(NC, h->tm, true);
      j.KB = (NC / nkb) << 9;
      j.NT = (j.RT + 15) / 16;
      j.UPR = j.KB >> 5;
      j.units = (size_t)nkb * j.NT * j.UPR;
      j.off = total;
      total += j.units * 512;
      jobs.push_back(j);
    }
    if (total) {
      if (hipMalloc((void**)&h->d_packed, total * 2) != hipSuccess) {
        h->d_packed = nullptr;
        return fail(YR_E_HIP, "yr_pk_pack_weights: cannot allocate %zu bytes", total * 2);
      }
      // one launch over every task's stream (the job table in a temporary
      // device buffer)
      std::vector<PackJob> pj(jobs.size());
      for (size_t i = 0; i < jobs.size(); i++) {
        const Job& j = jobs[i];
        TaskDesc& t = tasks[j.task];
        pj[i] = PackJob{t.w0, t.w1, h->d_packed + j.off, (unsigned long long)(j.off / 512), j.seg, j.RT, j.K, j.KB,
                        j.NT, j.UPR};
        t.w0 = h->d_packed + j.off;
        t.w1 = nullptr;
        t.packed = 1;
      }
      PackJob* d_jobs = nullptr;
      if (hipMalloc((void**)&d_jobs, sizeof(PackJob) * pj.size()) != hipSuccess) {
        (void)hipFree(h->d_packed);
        h->d_packed = nullptr;
        return fail(YR_E_HIP, "yr_pk_pack_weights: job table");
      }
      int rc = YR_OK;
      if (hipMemcpy(d_jobs, pj.data(), sizeof(PackJob) * pj.size(), hipMemcpyHostToDevice) != hipSuccess) {
        rc = fail(YR_E_HIP, "yr_pk_pack_weights: job table copy");
      } else {
        hipLaunchKernelGGL(pk_pack_kernel, dim3(4096), dim3(256), 0, 0, d_jobs, (int)pj.size(),
                           (unsigned long long)(total / 512));
        if (hipGetLastError() != hipSuccess || hipDeviceSynchronize() != hipSuccess)
          rc = fail(YR_E_HIP, "yr_pk_pack_weights: pack launch");
      }
      (void)hipFree(d_jobs);
      if (rc != YR_OK) {  // the launch keeps using the original weights
        (void)hipFree(h->d_packed);
        h->d_packed = nullptr;
        return rc;
      }
      if (bytes) *bytes = total * 2;
    }
  }
  if (hipMemcpy(h->d_tasks, tasks.data(), sizeof(TaskDesc) * tasks.size(), hipMemcpyHostToDevice) != hipSuccess)
    return fail(YR_E_HIP, "yr_pk_pack_weights: task copy");
  if (hipDeviceSynchronize() != hipSuccess) return fail(YR_E_HIP, "yr_pk_pack_weights: synchronize");
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
    return fail(YR_E_INVALID, "attention task %d: query rows per kv head beyond the op's split records, or more "
                "cached positions than the split's block budget", status4[3] - 1);
  return YR_OK;
}

int yr_pk_reset_status(yr_pk_handle* hp) {
  Handle* h = reinterpret_cast<Handle*>(hp);
  if (!h) return fail(YR_E_INVALID, "yr_pk_reset_status: null handle");
  // clear the flags and re-base the counters (a watchdog exit leaves them
  // short, the grid-barrier counter and split-K / multi-token attention
  // arrival tickets part-way)
  if (hipMemset(h->d_status, 0, sizeof(int) * 4) != hipSuccess) return fail(YR_E_HIP, "reset status");
  if (hipMemset(h->d_events, 0, sizeof(uint32_t) * (h->n_events + 1)) != hipSuccess)
    return fail(YR_E_HIP, "reset events");
  if (hipMemset(h->d_tickets, 0, sizeof(uint32_t) * (h->n_tickets + 1)) != hipSuccess)
    return fail(YR_E_HIP, "reset tickets");
  int rc = clear_tagged(h, nullptr);
  if (rc != YR_OK) return rc;
  if (hipDeviceSynchronize() != hipSuccess) return fail(YR_E_HIP, "reset status: synchronize");
  h->epoch = 0;
  return YR_OK;
}

void yr_pk_destroy(yr_pk_handle* hp) {
  Handle* h = reinterpret_cast<Handle*>(hp);
  if (!h) return;
  void* ptrs[] = {h->d_ops,     h->d_tasks,   h->d_qoff,    h->d_queue,  h->d_events,     h->d_triggers,
                  h->d_iters,   h->d_tickets, h->d_scratch, h->d_status, h->d_owned_meta, h->d_packed};
  for (void* p : ptrs)
    if (p) (void)hipFree(p);
  delete h;
}

}  // extern "C"
