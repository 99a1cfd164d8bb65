// GQA attention for gfx950: paged split-KV decode and causal prefill.
//
// Decode (HBM-bound, reads every cached K/V byte once):
//   grid = (kv splits, kv heads, batch), about one workgroup per CU; one
//   workgroup = 8 waves covers a chunk of tokens of one (sequence, kv head)
//   for all G = Hq/Hkv query heads of the group.  Q.K^T runs on MFMA 16x16x32
//   with the K rows as the B operand straight from HBM (16-byte loads, no
//   LDS); P.V runs on MFMA too, V going through LDS and coming back as B
//   fragments by transposing reads.  Every wave streams its own 32-token
//   blocks with an online softmax; the 8 waves merge in LDS, and
//   splits merge through the workspace with the last-arriving workgroup
//   (atomic ticket) writing the output.
//
// Prefill (MFMA-bound): flash attention, one workgroup per (64 query rows,
//   q head, batch); K tiles and transposed V tiles are staged in LDS, S = Q K^T
//   and O += P V both on MFMA 16x16x32, fp32 running max/sum per row.
#include <mutex>

#include "yr_common.h"
#include "attn_launch.h"

namespace yr {

constexpr float kLog2e = 1.4426950408889634f;

// ---------------------------------------------------------------- decode
// Streaming split-KV decode: grid = (splits, kv heads, batch) with about one
// workgroup per CU in total; a workgroup (8 waves) owns `chunk` tokens of one
// (sequence, kv head).  Its page ids are staged in LDS first, so no K/V load
// waits on a page-table load.  The waves stream 32-token blocks (K straight
// from HBM as MFMA B fragments, V through LDS), keep an online softmax per
// head row, and the 8 waves then the splits merge
// (splits through fp32 records, the last workgroup to arrive writing out).
constexpr int DEC_WAVES = 8;
constexpr int DEC_THREADS = DEC_WAVES * kWave;
constexpr int DEC_BLK = 32;        // tokens per wave block
constexpr int DEC_MAXPG = 4096;    // page ids staged per workgroup
constexpr int DEC_TARGET_WG = 256; // workgroups to aim for (one per CU)

struct DecodeArgs {
  const uint16_t* q;       // [B][Hq][D]
  const uint16_t* kc;      // [P][page][Hkv][D]
  const uint16_t* vc;
  const int32_t* kv_indptr;
  const int32_t* kv_indices;
  const int32_t* kv_len;
  uint16_t* out;           // [B][Hq][D]
  float* partial;          // [B][Hkv][splits][G][D + 2]
  uint32_t* tickets;       // [B][Hkv]
  int B, Hq, Hkv, page, splits, chunk;
  float scale_log2;        // log2(e) / sqrt(D)
};

#ifdef YR_DEC_PROF
__device__ uint64_t g_dec_prof[4096 * 8];
#define DPROF(i) \
  if (threadIdx.x == 0) g_dec_prof[(blockIdx.x + gridDim.x * (blockIdx.y + gridDim.y * blockIdx.z)) * 8 + (i)] = __builtin_amdgcn_s_memrealtime();
#else
#define DPROF(i)
#endif

// D = 128, G <= 16.  PG32 (page size a multiple of 32): a 32-token block
// lies in one page, whose id each wave reads with one scalar load when it
// issues the block (no page-table staging before the first K/V load);
// otherwise the split's page ids are staged in LDS first.
template <int DT, int G, bool PG32>
__global__ __launch_bounds__(DEC_THREADS) void gqa_decode_kernel(DecodeArgs a) {
  constexpr int D = 128;
  const int split = blockIdx.x, hk = blockIdx.y, b = blockIdx.z;
  const int tid = threadIdx.x, wave = tid / kWave, lane = tid % kWave;
  const int len = a.kv_len[b];
  const int c0 = split * a.chunk, c1 = min(len, c0 + a.chunk);
  const size_t tok_stride = (size_t)a.Hkv * D;  // elements between tokens in a page
  DPROF(0)

  constexpr int LDV = D + 8;       // padded V rows: transposing reads without bank conflicts
  constexpr int LDP = DEC_BLK + 8;
  static_assert(G * D * 4 <= DEC_BLK * LDV * 2, "wave's O must fit its V slot");
  __shared__ int s_pg[DEC_MAXPG];
  // per wave: the V block (then, after the loop, the wave's O as fp32 [G][D])
  __shared__ __attribute__((aligned(16))) uint16_t s_v[DEC_WAVES][DEC_BLK * LDV];
  __shared__ __attribute__((aligned(16))) uint16_t s_p[DEC_WAVES][16 * LDP];  // P as 16-bit [row][token]
  __shared__ float s_m[DEC_WAVES][G], s_l[DEC_WAVES][G];

  // ---- page ids of this split
  const int pg0 = c0 / a.page;
  const int npg = c1 > c0 ? (c1 - 1) / a.page - pg0 + 1 : 0;
  const int pbase = a.kv_indptr[b];
  if constexpr (!PG32)
    for (int i = tid; i < npg; i += DEC_THREADS) s_pg[i] = a.kv_indices[pbase + pg0 + i];
  // ---- Q as the MFMA A operand: row = head (lane%16 < G), k = d
  uint4 qf[4];
  {
    const int g = lane % 16;
    const uint16_t* qrow = a.q + ((size_t)b * a.Hq + (size_t)hk * G + (g < G ? g : 0)) * D;
#pragma unroll
    for (int s = 0; s < 4; s++) {
      qf[s] = ldg16(qrow + 32 * s + (lane / 16) * 8);
      if (g >= G) qf[s] = make_uint4(0, 0, 0, 0);
    }
  }
  __syncthreads();
  DPROF(1)

  const int nblk = c1 > c0 ? (c1 - c0 + DEC_BLK - 1) / DEC_BLK : 0;
  // element offset of token t (clamped into [c0, c1): finite data, masked)
  auto tok_off = [&](int t) __attribute__((always_inline)) -> size_t {
    t = min(max(t, c0), c1 - 1);
    const int pg = s_pg[t / a.page - pg0];
    return ((size_t)pg * a.page + t % a.page) * tok_stride + (size_t)hk * D;
  };
  struct Blk {
    uint4 k[2][4];  // [16-token tile j][k step s]: token 16 j + lane % 16, d = 32 s + 8 (lane / 16)
    uint4 v[8];     // token lane / 16 + 4 i, d = 8 (lane % 16)
  };
  // the page table through the scalar path (read-only for the launch)
  const __attribute__((address_space(4))) int32_t* kvi =
      reinterpret_cast<const __attribute__((address_space(4))) int32_t*>(reinterpret_cast<uintptr_t>(a.kv_indices));
  auto issue = [&](Blk& bk, int blk) __attribute__((always_inline)) {
    const int tb = __builtin_amdgcn_readfirstlane(c0 + blk * DEC_BLK);
    if constexpr (PG32) {
      // tokens tb .. tb + 31 (clamped to c1 - 1, the same block) share a page
      const int pg = kvi[pbase + tb / a.page];
      auto off32 = [&](int t) __attribute__((always_inline)) -> size_t {
        t = min(t, c1 - 1);
        return ((size_t)pg * a.page + t % a.page) * tok_stride + (size_t)hk * D;
      };
#pragma unroll
      for (int n = 0; n < 2; n++) {
        const size_t off = off32(tb + 16 * n + lane % 16) + (lane / 16) * 8;
#pragma unroll
        for (int s = 0; s < 4; s++) bk.k[n][s] = ldg16(a.kc + off + 32 * s);
      }
#pragma unroll
      for (int i = 0; i < 8; i++) bk.v[i] = ldg16(a.vc + off32(tb + lane / 16 + 4 * i) + (lane % 16) * 8);
    } else {
#pragma unroll
      for (int n = 0; n < 2; n++) {
        const size_t off = tok_off(tb + 16 * n + lane % 16) + (lane / 16) * 8;
#pragma unroll
        for (int s = 0; s < 4; s++) bk.k[n][s] = ldg16(a.kc + off + 32 * s);
      }
#pragma unroll
      for (int i = 0; i < 8; i++) bk.v[i] = ldg16(a.vc + tok_off(tb + lane / 16 + 4 * i) + (lane % 16) * 8);
    }
  };

  // online softmax state of rows 4 (lane / 16) + i; O in the MFMA C layout:
  // o[n][i] = row 4 (lane / 16) + i, dim 16 n + lane % 16
  float m_run[4], l_run[4];
#pragma unroll
  for (int i = 0; i < 4; i++) { m_run[i] = -INFINITY; l_run[i] = 0.f; }
  f32x4 o[D / 16];
#pragma unroll
  for (int n = 0; n < D / 16; n++) o[n] = f32x4{0.f, 0.f, 0.f, 0.f};
  uint16_t* vs = s_v[wave];
  uint16_t* ps = s_p[wave];

  // S = Q K^T and P V both on MFMA 16x16x32.  P goes through LDS as 16-bit
  // values (the A operand wants 8 consecutive tokens per lane), V through LDS
  // unchanged and comes back as B fragments by transposing reads.  Rows past G
  // hold finite values from zero Q rows and are never written out.
  auto consume = [&](const Blk& bk, int blk) __attribute__((always_inline)) {
    const int tb = c0 + blk * DEC_BLK;
#pragma unroll
    for (int i = 0; i < 8; i++)
      *reinterpret_cast<uint4*>(vs + (lane / 16 + 4 * i) * LDV + (lane % 16) * 8) = bk.v[i];
    f32x4 sc[2];
#pragma unroll
    for (int n = 0; n < 2; n++) {
      f32x4 c = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int s = 0; s < 4; s++) c = mfma16<DT>(qf[s], bk.k[n][s], c);
      sc[n] = c;
    }
    float alpha[4];
#pragma unroll
    for (int i = 0; i < 4; i++) {
      float mx = -INFINITY;
#pragma unroll
      for (int n = 0; n < 2; n++) {
        const float v = tb + 16 * n + lane % 16 < c1 ? sc[n][i] * a.scale_log2 : -INFINITY;
        sc[n][i] = v;
        mx = fmaxf(mx, v);
      }
#pragma unroll
      for (int o2 = 8; o2 > 0; o2 >>= 1) mx = fmaxf(mx, __shfl_xor(mx, o2, kWave));
      const float mnew = fmaxf(m_run[i], mx);
      alpha[i] = mnew == -INFINITY ? 1.f : exp2f(m_run[i] - mnew);
      float ls = 0.f;
      const int r = 4 * (lane / 16) + i;
#pragma unroll
      for (int n = 0; n < 2; n++) {
        const float p = round_to<DT>(mnew == -INFINITY ? 0.f : exp2f(sc[n][i] - mnew));
        ls += p;  // the sum uses the same rounded P as P V
        ps[r * LDP + 16 * n + lane % 16] = (uint16_t)st_elem<DT>(p);
      }
#pragma unroll
      for (int o2 = 8; o2 > 0; o2 >>= 1) ls += __shfl_xor(ls, o2, kWave);
      l_run[i] = l_run[i] * alpha[i] + ls;
      m_run[i] = mnew;
    }
    // LDS operations of one wave complete in order; the asm keeps the
    // compiler from moving the reads above the writes.
    asm volatile("" ::: "memory");
    const uint4 pa = *reinterpret_cast<const uint4*>(ps + (lane % 16) * LDP + (lane / 16) * 8);
#pragma unroll
    for (int n = 0; n < D / 16; n++) {
#pragma unroll
      for (int i = 0; i < 4; i++) o[n][i] *= alpha[i];
      o[n] = mfma16<DT>(pa, b_frag(vs + 16 * n, LDV, 0, lane), o[n]);
    }
    asm volatile("" ::: "memory");  // the next block's writes stay after these reads
  };

  // Wave w takes blocks w, w + 8, ... (a fixed order, so results do not
  // depend on timing).  One block in flight per wave: with every workgroup
  // resident that is ~64 MiB queued at once, and deeper queues only lengthen
  // the tail.
  int cur = wave;
  if (cur < nblk) {
    Blk bk;
    issue(bk, cur);
    bool first = true;
    for (;;) {
      const int nxt = cur + DEC_WAVES;
      consume(bk, cur);
      if (first) DPROF(2)
      first = false;
      if (nxt >= nblk) break;
      issue(bk, nxt);
      cur = nxt;
    }
  }

  DPROF(3)
  // ---- the 8 waves merge through LDS (O over the wave's own V slot)
  float* os = reinterpret_cast<float*>(vs);
#pragma unroll
  for (int i = 0; i < 4; i++) {
    const int r = 4 * (lane / 16) + i;
    if (r < G) {
#pragma unroll
      for (int n = 0; n < D / 16; n++) os[r * D + 16 * n + lane % 16] = o[n][i];
      if ((lane % 16) == 0) {
        s_m[wave][r] = m_run[i];
        s_l[wave][r] = l_run[i];
      }
    }
  }
  __syncthreads();

  const int REC = D + 2;
  float* rec_base = a.partial + (((size_t)b * a.Hkv + hk) * a.splits) * G * REC;
  for (int idx = tid; idx < G * D; idx += DEC_THREADS) {
    const int g = idx / D, d = idx % D;
    float M = -INFINITY;
#pragma unroll
    for (int w = 0; w < DEC_WAVES; w++) M = fmaxf(M, s_m[w][g]);
    float L = 0.f, O = 0.f;
#pragma unroll
    for (int w = 0; w < DEC_WAVES; w++) {
      const float f = s_m[w][g] == -INFINITY ? 0.f : exp2f(s_m[w][g] - M);
      L += s_l[w][g] * f;
      O += reinterpret_cast<const float*>(s_v[w])[g * D + d] * f;
    }
    if (a.splits == 1) {
      a.out[((size_t)b * a.Hq + (size_t)hk * G + g) * D + d] = (uint16_t)st_elem<DT>(L > 0.f ? O / L : 0.f);
    } else {
      float* rec = rec_base + ((size_t)split * G + g) * REC;
      st_agent(rec + d, O);
      if (d == 0) {
        st_agent(rec + D, M);
        st_agent(rec + D + 1, L);
      }
    }
  }
  DPROF(4)
  if (a.splits == 1) return;

  // ---- split merge by the last workgroup of this (b, hk): every record in
  // flight at once (one thread per (g, d, split lane j of P))
  if (!arrive_last(&a.tickets[b * a.Hkv + hk], a.splits)) return;
  DPROF(5)
  for (int idx = tid; idx < G * D; idx += DEC_THREADS) {
    const int g = idx / D, d = idx % D;
    float M = -INFINITY, L = 0.f, O = 0.f;
    for (int s0 = 0; s0 < a.splits; s0 += 16) {
      float mv[16], lv[16], ov[16];
#pragma unroll
      for (int u = 0; u < 16; u++) {
        if (s0 + u < a.splits) {
          const float* rec = rec_base + ((size_t)(s0 + u) * G + g) * REC;
          mv[u] = ld_agent(rec + D);
          lv[u] = ld_agent(rec + D + 1);
          ov[u] = ld_agent(rec + d);
        } else {
          mv[u] = -INFINITY;
          lv[u] = 0.f;
          ov[u] = 0.f;
        }
      }
      float mb = M;
#pragma unroll
      for (int u = 0; u < 16; u++) mb = fmaxf(mb, mv[u]);
      const float f0 = M == -INFINITY ? 0.f : exp2f(M - mb);
      L *= f0;
      O *= f0;
#pragma unroll
      for (int u = 0; u < 16; u++) {
        const float f = mv[u] == -INFINITY ? 0.f : exp2f(mv[u] - mb);
        L += lv[u] * f;
        O += ov[u] * f;
      }
      M = mb;
    }
    a.out[((size_t)b * a.Hq + (size_t)hk * G + g) * D + d] = (uint16_t)st_elem<DT>(L > 0.f ? O / L : 0.f);
  }
  DPROF(6)
}

// Splits per (sequence, kv head): about DEC_TARGET_WG workgroups in total,
// each split a whole number of 32-token blocks.
struct DecPlan {
  int splits, chunk;
};
// A split also spans at most DEC_MAXPG - 2 pages (the staged page ids).
static DecPlan dec_plan(int batch, int hkv, int max_len, int page) {
  DecPlan p;
  const int pairs = batch * hkv > 0 ? batch * hkv : 1;
  int sp = (DEC_TARGET_WG + pairs - 1) / pairs;
  const int maxsp = (max_len + DEC_BLK - 1) / DEC_BLK;
  sp = sp < 1 ? 1 : sp > maxsp ? maxsp : sp;
  p.chunk = ((max_len + sp - 1) / sp + DEC_BLK - 1) / DEC_BLK * DEC_BLK;
  const long cap = ((long)(DEC_MAXPG - 2) * (page > 0 ? page : 1)) / DEC_BLK * DEC_BLK;
  if (p.chunk > cap) p.chunk = (int)cap;
  p.splits = (max_len + p.chunk - 1) / p.chunk;
  return p;
}

// ---------------------------------------------------------------- prefill
// Flash attention computed transposed: S^T = K Q^T and O^T += V^T P^T on
// MFMA 16x16x32, so a lane of the S^T accumulator holds one query row (its
// column) and 16 tokens of each 64-token tile:
//   * the softmax row max / sum is an in-register reduction plus two shuffles;
//   * P^T is the B operand of P V straight from registers: MFMA only needs the
//     k order of A and B to agree, so lane group h's k slots 8h + 4j + i carry
//     tokens 16 j + 4h + i of each 32-token step (j, i < 2, 4);
//   * V^T (the A operand) comes from the row-major V tile in LDS by
//     transposing reads, addressed for that same token order.
// A workgroup (4 waves x 16 query rows) serves HPW heads of one kv group, so
// each K / V fragment read from LDS feeds HPW MFMAs.  K / V tiles are double
// buffered in LDS (one barrier per tile).  For causal attention a workgroup
// takes the query blocks i and N - 1 - i, so every workgroup does the same
// amount of work.
constexpr int PF_QROWS = 64;             // query rows per block (4 row waves x 16)
constexpr int PF_KT = 64;                // kv tokens per tile
constexpr int PF_NB = PF_KT / 16;        // 16-token MFMA blocks per tile
constexpr float kLazy = 8.f;             // running-max slack (log2 units)

struct PrefillArgs {
  const uint16_t* q;  // [B] x [Sq] rows x [Hq][D]: row r of batch b at b q_bs + r q_ld
  const uint16_t* k;  // [B] x [Sk] rows x [Hkv][D]: b kv_bs + r kv_ld
  const uint16_t* v;
  uint16_t* o;        // like q: b o_bs + r o_ld
  long long q_bs, kv_bs, o_bs;  // batch strides (elements)
  int q_ld, kv_ld, o_ld;        // row strides (elements)
  int B, Sq, Sk, Hq, Hkv, causal, nblk;  // causal needs Sq == Sk
  int paired;  // blocks (i, nblk - 1 - i) per workgroup (causal)
  int npair, ngrp, nwg;  // workgroups per (batch, head group); head groups; total
  float scale_log2;
};

// 4 consecutive 16-bit elements from LDS, transposed across each 16-lane group
__device__ __forceinline__ uint2 lds_tr4(const uint16_t* p) {
  const v4i16 r = __builtin_amdgcn_ds_read_tr16_b64_v4i16(const_cast<lds_v4i16*>(
      reinterpret_cast<const lds_v4i16*>(reinterpret_cast<const __attribute__((address_space(3))) uint16_t*>(
          reinterpret_cast<uintptr_t>(p)))));
  return __builtin_bit_cast(uint2, r);
}

// max over lanes l and l ^ 16 (l ^ 32): a permlane swap of the value with
// itself hands each 16-lane row its partner row, in registers (no LDS trip)
__device__ __forceinline__ float max_xor16(float x) {
  const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float max_xor32(float x) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}

// 16-byte chunk permutation of a 256-byte LDS row: bits 1..3 = row % 8,
// bit 0 = (row / 8) % 2.  16 consecutive rows get 16 distinct values (K
// fragment reads, one chunk column over 16 rows), and 8 rows starting at a
// multiple of 8 keep bit 0 fixed (transposing V reads, chunk pairs 2c, 2c + 1).
__device__ __forceinline__ int pf_swz(int row) { return ((row & 7) << 1) | ((row >> 3) & 1); }
// K tiles: chunk permutation row % 16.  A 16-byte LDS read is served 8 lanes
// per 128 bytes: the K fragment read (lanes = 16 consecutive rows, one chunk
// column) then gives any 8 consecutive lanes 8 distinct chunks modulo 8,
// which pf_swz (even chunks for rows 0..7) does not (measured: all bank
// conflicts of the kernel were K reads)
__device__ __forceinline__ int pk_swz(int row) { return row & 15; }

// 16 bytes per lane from global memory straight into LDS: lane l's data
// lands at lds_base + 16 l (lds_base wave-uniform)
__device__ __forceinline__ void lds_load16(const uint16_t* g, uint16_t* lds_base) {
  __builtin_amdgcn_global_load_lds(
      (const __attribute__((address_space(1))) void*)(g),
      reinterpret_cast<__attribute__((address_space(3))) void*>(
          reinterpret_cast<__attribute__((address_space(3))) char*>(reinterpret_cast<uintptr_t>(lds_base))),
      16, 0, 0);
}

// HPW heads per wave, HG head groups (of 4 row waves) per workgroup
template <int DT, int HPW, int HG>
__global__ __launch_bounds__(256 * HG) void gqa_prefill_kernel(PrefillArgs a) {
  constexpr int D = 128;
  // K / V tiles: unpadded 256-byte rows whose 16-byte chunks are permuted by
  // row (pk_swz for K, pf_swz for V); they arrive by direct global -> LDS
  // loads (no registers)
  // separate objects per stage: the compiler then knows that reads of one
  // stage do not wait for the direct loads still filling the other
  __shared__ __attribute__((aligned(16))) uint16_t sk0[PF_KT * D], sk1[PF_KT * D];
  __shared__ __attribute__((aligned(16))) uint16_t sv0[PF_KT * D], sv1[PF_KT * D];
  // Q^T fragments in fragment order (lane l's 16 bytes at 16 l: no bank
  // conflicts), re-read by every S^T block instead of held in registers
  __shared__ uint4 sq[4 * HG][HPW][4][kWave];

  // workgroup i runs on XCD i % 8; work items are numbered so that one
  // XCD's share is contiguous, i.e. whole kv heads whose K / V stay in that
  // XCD's L2
  const int id = blockIdx.x;
  const int w = a.nwg % 8 == 0 ? (id % 8) * (a.nwg / 8) + id / 8 : id;
  const int pair = w % a.npair, hg = (w / a.npair) % a.ngrp, b = w / (a.npair * a.ngrp);
  const int G = a.Hq / a.Hkv;
  const int tid = threadIdx.x, lane = tid % kWave;
  const int wv = __builtin_amdgcn_readfirstlane(tid / kWave);  // wave index, uniform
  const int rw = wv % 4;                                       // row wave
  const int h0 = (hg * HG + wv / 4) * HPW;                     // this wave's first head
  const int hk = hg * HG * HPW / G;  // the workgroup's heads share one kv head (G % (HG HPW) == 0)
  const int col = lane % 16, grp = lane / 16;
  const size_t kstride = (size_t)a.kv_ld;
  const uint16_t* kbase = a.k + (size_t)b * a.kv_bs + (size_t)hk * D;
  const uint16_t* vbase = a.v + (size_t)b * a.kv_bs + (size_t)hk * D;
  // staging: wave w fills rows RPW w .. RPW w + RPW - 1, four rows per load;
  // lane l writes physical chunk l % 16 of row 4 u + l / 16, i.e. source
  // chunk (l % 16) ^ pk_swz(row) (K) or ^ pf_swz(row) (V)
  constexpr int RPW = PF_KT / (4 * HG);
  const int st_row0 = RPW * wv + lane / 16;
  // per-lane byte offsets of the staged chunks within a tile (rows of a tile
  // below S), and the element offsets of the K fragment reads (block n adds
  // 16 n D: pk_swz of row 16 n + col does not depend on n)
  // (V tiles' offsets are formed per fetch: one register array fewer)
  uint32_t foffk[RPW / 4];
#pragma unroll
  for (int u = 0; u < RPW / 4; u++) {
    const int row = st_row0 + 4 * u;
    foffk[u] = 2u * (uint32_t)(row * (int)kstride + 8 * ((lane % 16) ^ pk_swz(row)));
  }
  uint32_t koff[4];
#pragma unroll
  for (int s = 0; s < 4; s++) koff[s] = col * D + 8 * ((4 * s + grp) ^ pk_swz(col));
  // V^T fragment reads: lane 4e + q of group grp reads tokens 32 m + 16 j +
  // 4 grp + e, d 16 dt + 4 q .. +3 (q = 2 qc + qh / 4); pf_swz of those rows
  // depends on neither m nor j, so (m, j) add 16 (2 m + j) D
  uint32_t voff[D / 16];
  {
    const int e = col / 4, qc = (col % 4) / 2, qh = 4 * (col % 2), r0 = 4 * grp + e;
#pragma unroll
    for (int dt = 0; dt < D / 16; dt++) voff[dt] = r0 * D + 8 * ((2 * dt + qc) ^ pf_swz(r0)) + qh;
  }

  for (int pass = 0; pass < (a.paired ? 2 : 1); pass++) {
    const int blk = pass == 0 ? pair : a.nblk - 1 - pair;
    if (pass == 1 && blk <= pair) break;  // the middle block of an odd count runs once
    const int q0 = blk * PF_QROWS + rw * 16;  // this wave's first query row
    const int qr = q0 + col;                    // this lane's query row
    // Q^T as the B operand: column = query row, k = d 32 s + 8 grp .. +7
#pragma unroll
    for (int hh = 0; hh < HPW; hh++) {
      const uint16_t* qrow = a.q + (size_t)b * a.q_bs + (size_t)min(qr, a.Sq - 1) * a.q_ld + (size_t)(h0 + hh) * D;
#pragma unroll
      for (int s = 0; s < 4; s++) sq[wv][hh][s][lane] = ldg16(qrow + 32 * s + 8 * grp);
    }
    f32x4 acc[HPW][D / 16];  // O^T: rows d 16 dt + 4 grp + i, column = query row
#pragma unroll
    for (int hh = 0; hh < HPW; hh++)
#pragma unroll
      for (int dt = 0; dt < D / 16; dt++) acc[hh][dt] = f32x4{0.f, 0.f, 0.f, 0.f};
    float m_i[HPW], l_i[HPW];
#pragma unroll
    for (int hh = 0; hh < HPW; hh++) {
      m_i[hh] = -INFINITY;
      l_i[hh] = 0.f;
    }

    const int kv_end = a.causal ? min(a.Sk, (blk + 1) * PF_QROWS) : a.Sk;
    const int ntile = (kv_end + PF_KT - 1) / PF_KT;
    // tiles that need no mask: below every query row of the block and
    // entirely inside the sequence
    const int nfull = a.causal ? min(ntile, blk * PF_QROWS / PF_KT) : a.Sk / PF_KT;
    // causal: the last tile holding a key at or below this wave's rows
    const int tw_end = a.causal ? min(ntile, (q0 + 15) / PF_KT + 1) : ntile;
    // IS_K: the K tile's chunk permutation (pk_swz), else V's (pf_swz)
    auto fetch = [&](int t, const uint16_t* base, uint16_t* dst, auto is_k_c) __attribute__((always_inline)) {
      constexpr bool IS_K = decltype(is_k_c)::value;
      const char* tb = reinterpret_cast<const char*>(base + (size_t)t * PF_KT * kstride);  // uniform
      const bool whole = (t + 1) * PF_KT <= a.Sk;
#pragma unroll
      for (int u = 0; u < RPW / 4; u++) {
        const int row = st_row0 + 4 * u;
        uint32_t off;
        if constexpr (IS_K) off = foffk[u];
        else off = 2u * (uint32_t)(row * (int)kstride + 8 * ((lane % 16) ^ pf_swz(row)));
        if (!whole) {  // last tile: rows past Sk re-read token Sk - 1 (masked)
          const int r = min(t * PF_KT + row, a.Sk - 1) - t * PF_KT;
          off = 2u * (uint32_t)(r * (int)kstride + 8 * ((lane % 16) ^ (IS_K ? pk_swz(row) : pf_swz(row))));
        }
        lds_load16(reinterpret_cast<const uint16_t*>(tb + off), dst + (RPW * wv + 4 * u) * D);
      }
    };
    // S^T = K Q^T: 4 blocks of 16 tokens; lane holds tokens t0 + 16 n + 4 grp + i
    using Scores = f32x4[HPW][PF_NB];
    using PFrag = uint4[HPW][PF_NB / 2];
    auto qk = [&](const uint16_t* kt, Scores& sc) __attribute__((always_inline)) {
#pragma unroll
      for (int n = 0; n < PF_NB; n++) {
        uint4 kf[4];
#pragma unroll
        for (int s = 0; s < 4; s++) kf[s] = *reinterpret_cast<const uint4*>(&kt[koff[s] + 16 * n * D]);
#pragma unroll
        for (int hh = 0; hh < HPW; hh++) {
          f32x4 c = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
          for (int s = 0; s < 4; s++) c = mfma16<DT>(kf[s], sq[wv][hh][s][lane], c);
          sc[hh][n] = c;
        }
      }
    };
    // online softmax of this lane's query row over tile t, in two parts so
    // that S(t + 1) can be issued between them.  smax: mask (EDGE: the tile
    // crosses the causal diagonal or the end of the sequence), row max, O
    // rescale.  The running max only moves when it grows by more than kLazy
    // (log2 units): P stays <= 2^kLazy, exact after the final 1 / l, and the
    // rescale is skipped by the whole wave on most tiles.  Scores stay
    // unscaled: the max commutes with the positive scale, which is folded
    // into the exponent's fma.
    auto smax = [&](int t, Scores& sc, auto edge_c) __attribute__((always_inline)) {
      constexpr bool EDGE = decltype(edge_c)::value;
      const int t0 = t * PF_KT;
#pragma unroll
      for (int hh = 0; hh < HPW; hh++) {
        if (EDGE) {
#pragma unroll
          for (int n = 0; n < PF_NB; n++)
#pragma unroll
            for (int i = 0; i < 4; i++) {
              const int tok = t0 + 16 * n + 4 * grp + i;
              if (tok >= a.Sk || (a.causal && tok > qr)) sc[hh][n][i] = -INFINITY;
            }
        }
        float mx = -INFINITY;
#pragma unroll
        for (int n = 0; n < PF_NB; n++)
#pragma unroll
          for (int i = 0; i < 4; i++) mx = fmaxf(mx, sc[hh][n][i]);
        mx = max_xor16(mx);
        mx = max_xor32(mx);
        mx *= a.scale_log2;
        const bool grow = mx > m_i[hh] + kLazy;
        if (__builtin_amdgcn_ballot_w64(grow)) {
          const float mnew = grow ? mx : m_i[hh];
          const float alpha = m_i[hh] == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(m_i[hh] - mnew);
          m_i[hh] = mnew;
          l_i[hh] *= alpha;
#pragma unroll
          for (int dt = 0; dt < D / 16; dt++) acc[hh][dt] *= alpha;
        }
      }
    };
    // sexp: P = exp2(s scale - m) as the B operands of P V, row sums in l
    auto sexp = [&](const Scores& sc, PFrag& pb) __attribute__((always_inline)) {
#pragma unroll
      for (int hh = 0; hh < HPW; hh++) {
        const float mref = m_i[hh] == -INFINITY ? 0.f : m_i[hh];  // all -inf so far: P = 0
        float ls = 0.f;
        float pv[PF_NB][4];
#pragma unroll
        for (int n = 0; n < PF_NB; n++)
#pragma unroll
          for (int i = 0; i < 4; i++) {
            const float p = __builtin_amdgcn_exp2f(fmaf(sc[hh][n][i], a.scale_log2, -mref));
            pv[n][i] = p;
            ls += p;
          }
        l_i[hh] += ls;  // per lane; the four lane groups add up at the end
        // k slot 8 grp + 4 j + i of step m <-> token 32 m + 16 j + 4 grp + i
#pragma unroll
        for (int m = 0; m < PF_NB / 2; m++)
          pb[hh][m] = make_uint4(pack2<DT>(pv[2 * m][0], pv[2 * m][1]), pack2<DT>(pv[2 * m][2], pv[2 * m][3]),
                                 pack2<DT>(pv[2 * m + 1][0], pv[2 * m + 1][1]),
                                 pack2<DT>(pv[2 * m + 1][2], pv[2 * m + 1][3]));
      }
    };
    // O^T += V^T P^T.  V^T fragment (rows d 16 dt + col, k slots as above):
    // lane 4e + q of group grp reads tokens 32 m + 16 j + 4 grp + e, d 16 dt
    // + 4 q .. +3; the transposing read hands lane col its d.
    auto pv = [&](const uint16_t* vt, const PFrag& pb) __attribute__((always_inline)) {
#pragma unroll
      for (int m = 0; m < PF_NB / 2; m++)
#pragma unroll
        for (int dt = 0; dt < D / 16; dt++) {
          const uint2 lo = lds_tr4(&vt[voff[dt] + 32 * m * D]);
          const uint2 hi = lds_tr4(&vt[voff[dt] + (32 * m + 16) * D]);
          const uint4 vf = make_uint4(lo.x, lo.y, hi.x, hi.y);
#pragma unroll
          for (int hh = 0; hh < HPW; hh++) acc[hh][dt] = mfma16<DT>(vf, pb[hh][m], acc[hh][dt]);
        }
    };
    // Software pipeline: step t computes S(t + 1) on MFMA while the softmax
    // of S(t) runs on VALU, then P(t) V(t).  K runs one tile ahead of V, so
    // step t reads K(t + 1) and V(t) while K(t + 2) and V(t + 1) stream into
    // the buffers whose previous contents step t - 1 finished reading.
    Scores sA, sB;
    PFrag pb;
    __syncthreads();  // the previous pass's last tiles have been read by every wave
    fetch(0, kbase, sk0, std::true_type{});
    fetch(0, vbase, sv0, std::false_type{});
    if (ntile > 1) fetch(1, kbase, sk1, std::true_type{});
    wait_vm();
    __syncthreads();
    qk(sk0, sA);
    __syncthreads();  // every wave is done with K(0) before K(2) replaces it
    // a step with a following tile (t + 1 < ntile) and no mask
    auto step = [&](int t, const uint16_t* kq, const uint16_t* vp, uint16_t* nk, uint16_t* nv, Scores& scur,
                    Scores& snext) __attribute__((always_inline)) {
      if (t + 2 < ntile) fetch(t + 2, kbase, nk, std::true_type{});
      fetch(t + 1, vbase, nv, std::false_type{});
      smax(t, scur, std::false_type{});
      qk(kq, snext);
      sexp(scur, pb);
      pv(vp, pb);
      wait_vm();  // K(t + 2) and V(t + 1) have landed in LDS
      __syncthreads();
    };
    // the last tile: masked, nothing to fetch or prefetch
    auto last = [&](int t, const uint16_t* vp, Scores& scur) __attribute__((always_inline)) {
      if (t < tw_end) {
        smax(t, scur, std::true_type{});
        sexp(scur, pb);
        pv(vp, pb);
      }
    };
    // tiles below nfull need no mask; the last tile always takes the masked
    // path (for causal blocks it is the diagonal one)
    const int nstep = min(nfull, ntile - 1);
    int t = 0;
    for (; t + 1 < nstep; t += 2) {
      step(t, sk1, sv0, sk0, sv1, sA, sB);
      step(t + 1, sk0, sv1, sk1, sv0, sB, sA);
    }
    if (t < nstep) {
      step(t, sk1, sv0, sk0, sv1, sA, sB);
      t++;
    }
    // t == ntile - 1 here: ntile - nfull <= 1 (non-causal: floor and ceiling
    // of S / PF_KT; causal: the block's rows start at blk PF_QROWS, so tiles
    // below blk PF_QROWS / PF_KT are full and one more reaches its last row)
    if (t % 2 == 0) last(t, sv0, sA);
    else last(t, sv1, sB);
    // O[query row][d 16 dt + 4 grp + i]
#pragma unroll
    for (int hh = 0; hh < HPW; hh++) {
      l_i[hh] += __shfl_xor(l_i[hh], 16, kWave);
      l_i[hh] += __shfl_xor(l_i[hh], 32, kWave);
    }
    if (qr < a.Sq) {
#pragma unroll
      for (int hh = 0; hh < HPW; hh++) {
        const float inv = l_i[hh] > 0.f ? 1.f / l_i[hh] : 0.f;
        uint16_t* orow = a.o + (size_t)b * a.o_bs + (size_t)qr * a.o_ld + (size_t)(h0 + hh) * D;
#pragma unroll
        for (int dt = 0; dt < D / 16; dt++) {
          const f32x4 v = acc[hh][dt];
          *reinterpret_cast<uint2*>(orow + 16 * dt + 4 * grp) =
              make_uint2(pack2<DT>(v[0] * inv, v[1] * inv), pack2<DT>(v[2] * inv, v[3] * inv));
        }
      }
    }
  }
}

// ---------------------------------------------------------------- argmax
// One workgroup per row; lowest index wins ties.
template <int DT>
__global__ __launch_bounds__(256) void argmax_kernel(const uint16_t* x, int64_t* out, int n, int n_valid) {
  const int row = blockIdx.x;
  const uint16_t* xr = x + (size_t)row * n;
  float best = -INFINITY;
  int bi = 0x7fffffff;
  for (int i = threadIdx.x; i < n_valid; i += blockDim.x) {
    float v = ld_elem<DT>(xr[i]);
    if (v > best || (v == best && i < bi)) {
      best = v;
      bi = i;
    }
  }
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) {
    float ov = __shfl_xor(best, o, kWave);
    int oi = __shfl_xor(bi, o, kWave);
    if (ov > best || (ov == best && oi < bi)) {
      best = ov;
      bi = oi;
    }
  }
  __shared__ float sv[4];
  __shared__ int si[4];
  int w = threadIdx.x / kWave;
  if (threadIdx.x % kWave == 0) {
    sv[w] = best;
    si[w] = bi;
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    for (int k = 1; k < (int)(blockDim.x / kWave); k++)
      if (sv[k] > best || (sv[k] == best && si[k] < bi)) {
        best = sv[k];
        bi = si[k];
      }
    out[row] = bi == 0x7fffffff ? -1 : bi;
  }
}

}  // namespace yr

using namespace yr;

extern "C" {

size_t yr_hip_gqa_decode_workspace(int batch, int hq, int hkv, int d, int max_kv_len, int page_size) {
  int sp = dec_plan(batch, hkv, max_kv_len, page_size).splits;
  if (sp <= 1 || hkv <= 0) return 0;
  int G = hq / hkv;
  return kTicketBytes + (size_t)batch * hkv * sp * G * (d + 2) * sizeof(float);
}

}  // extern "C"

// Shape / dtype checks of a paged decode call (everything but the workspace).
int yr::gqa_decode_check(const char* nm, const void* q, const void* k_cache, const void* v_cache,
                         const int32_t* kv_indptr, const int32_t* kv_indices, const int32_t* kv_len, const void* out,
                         int batch, int hq, int hkv, int d, int page_size, int max_kv_len, int dtype) {
  if (!q || !k_cache || !v_cache || !kv_indptr || !kv_indices || !kv_len || !out)
    return fail(YR_E_INVALID, "%s: null pointer", nm);
  if (batch <= 0 || hkv <= 0 || hq % hkv) return fail(YR_E_INVALID, "%s: hq must be a multiple of hkv", nm);
  if (d != 128) return fail(YR_E_INVALID, "%s: head_dim %d unsupported (128)", nm, d);
  const int G = hq / hkv;
  if (G != 1 && G != 2 && G != 4 && G != 8 && G != 16) return fail(YR_E_INVALID, "%s: group size %d", nm, G);
  if (page_size <= 0) return fail(YR_E_INVALID, "%s: bad page size", nm);
  if (dtype != YR_DTYPE_F16 && dtype != YR_DTYPE_BF16) return fail(YR_E_INVALID, "%s: dtype", nm);
  if (max_kv_len <= 0) return fail(YR_E_INVALID, "%s: max_kv_len must be > 0", nm);
  if (batch * hkv > kMaxTickets) return fail(YR_E_INVALID, "%s: batch * hkv too large", nm);
  const DecPlan dp = dec_plan(batch, hkv, max_kv_len, page_size);
  if (dp.chunk / page_size + 2 > DEC_MAXPG)
    return fail(YR_E_INVALID, "%s: %d pages per split exceed %d (page_size too small)", nm, dp.chunk / page_size + 2,
                DEC_MAXPG);
  return YR_OK;
}

// The decode launch shared by the workspace and the no-allocation entry
// points: checks the shape, plans the splits and launches.
int yr::gqa_decode_launch(const char* nm, const void* q, const void* k_cache, const void* v_cache,
                             const int32_t* kv_indptr, const int32_t* kv_indices, const int32_t* kv_len, void* out,
                             int batch, int hq, int hkv, int d, int page_size, int max_kv_len, int dtype,
                             void* workspace, size_t workspace_bytes, hipStream_t st, float scale) {
  int rc = gqa_decode_check(nm, q, k_cache, v_cache, kv_indptr, kv_indices, kv_len, out, batch, hq, hkv, d,
                            page_size, max_kv_len, dtype);
  if (rc != YR_OK) return rc;
  const int G = hq / hkv;
  size_t need = yr_hip_gqa_decode_workspace(batch, hq, hkv, d, max_kv_len, page_size);
  if (need > workspace_bytes || (need && !workspace))
    return fail(YR_E_WORKSPACE, "%s: workspace %zu < %zu", nm, workspace_bytes, need);
  DecodeArgs a;
  a.q = (const uint16_t*)q;
  a.kc = (const uint16_t*)k_cache;
  a.vc = (const uint16_t*)v_cache;
  a.kv_indptr = kv_indptr;
  a.kv_indices = kv_indices;
  a.kv_len = kv_len;
  a.out = (uint16_t*)out;
  a.B = batch;
  a.Hq = hq;
  a.Hkv = hkv;
  a.page = page_size;
  const DecPlan dp = dec_plan(batch, hkv, max_kv_len, page_size);
  a.splits = dp.splits;
  a.chunk = dp.chunk;
  a.tickets = (uint32_t*)workspace;
  a.partial = need ? (float*)((char*)workspace + kTicketBytes) : nullptr;
  if (!(scale > 0.f)) return fail(YR_E_INVALID, "%s: scale must be positive", nm);
  a.scale_log2 = kLog2e * scale;
  dim3 grid(a.splits, hkv, batch);
#define YR_DEC(G_)                                                                                        \
  if (G == G_) {                                                                                          \
    if (page_size % DEC_BLK == 0) {                                                                       \
      if (dtype == YR_DTYPE_F16) hipLaunchKernelGGL((gqa_decode_kernel<DT_F16, G_, true>), grid, dim3(DEC_THREADS), 0, st, a); \
      else hipLaunchKernelGGL((gqa_decode_kernel<DT_BF16, G_, true>), grid, dim3(DEC_THREADS), 0, st, a);   \
    } else {                                                                                              \
      if (dtype == YR_DTYPE_F16) hipLaunchKernelGGL((gqa_decode_kernel<DT_F16, G_, false>), grid, dim3(DEC_THREADS), 0, st, a); \
      else hipLaunchKernelGGL((gqa_decode_kernel<DT_BF16, G_, false>), grid, dim3(DEC_THREADS), 0, st, a);  \
    }                                                                                                     \
  }
  YR_DEC(1) YR_DEC(2) YR_DEC(4) YR_DEC(8) YR_DEC(16)
#undef YR_DEC
  YR_CHECK_LAUNCH(nm);
  return YR_OK;
}

// The prefill launch behind yr_hip_gqa_prefill and the kernel-graph
// attention: q rows Sq, kv rows Sk (causal needs Sq == Sk), explicit batch /
// row strides in elements, softmax scale `scale` (scores are multiplied by
// it before the exponential).
int yr::prefill_launch(const char* nm, const void* q, const void* k, const void* v, void* out, int batch, int sq, int sk,
                   int hq, int hkv, int d, int causal, int dtype, long long q_bs, int q_ld, long long kv_bs, int kv_ld,
                   long long o_bs, int o_ld, float scale, hipStream_t st) {
  if (!q || !k || !v || !out) return fail(YR_E_INVALID, "%s: null pointer", nm);
  if (batch <= 0 || sq <= 0 || sk <= 0 || hkv <= 0 || hq % hkv) return fail(YR_E_INVALID, "%s: bad shape", nm);
  if (d != 128) return fail(YR_E_INVALID, "%s: head_dim %d unsupported (128)", nm, d);
  if (dtype != YR_DTYPE_F16 && dtype != YR_DTYPE_BF16) return fail(YR_E_INVALID, "%s: dtype", nm);
  if (causal && sq != sk) return fail(YR_E_INVALID, "%s: causal attention needs as many query as kv rows", nm);
  if (q_ld % 8 || kv_ld % 8 || o_ld % 8 || q_bs % 8 || kv_bs % 8 || o_bs % 8 || q_ld < hq * d || kv_ld < hkv * d ||
      o_ld < hq * d)
    return fail(YR_E_INVALID, "%s: strides must be multiples of 8 elements and cover a row", nm);
  if ((long long)kv_ld * 64 * 2 >= (1ll << 31)) return fail(YR_E_INVALID, "%s: kv row stride too large", nm);
  if (!(scale > 0.f)) return fail(YR_E_INVALID, "%s: scale must be positive", nm);
  PrefillArgs a;
  a.q = (const uint16_t*)q;
  a.k = (const uint16_t*)k;
  a.v = (const uint16_t*)v;
  a.o = (uint16_t*)out;
  a.q_bs = q_bs;
  a.kv_bs = kv_bs;
  a.o_bs = o_bs;
  a.q_ld = q_ld;
  a.kv_ld = kv_ld;
  a.o_ld = o_ld;
  a.B = batch;
  a.Sq = sq;
  a.Sk = sk;
  a.Hq = hq;
  a.Hkv = hkv;
  a.causal = causal ? 1 : 0;
  a.nblk = (sq + PF_QROWS - 1) / PF_QROWS;
  a.scale_log2 = kLog2e * scale;
  // heads per workgroup: 2 when the group size allows (two groups of 4 row
  // waves sharing each K / V tile), one head per wave
  const int G = hq / hkv;
#ifndef YR_PF_CFG
#define YR_PF_CFG 2
#endif
  const int hpw = (YR_PF_CFG == 0 || YR_PF_CFG == 3) && G % 2 == 0 ? 2 : 1;
  const int hgw = (YR_PF_CFG >= 2) && (G / hpw) % 2 == 0 ? 2 : 1;
  a.paired = a.causal;
  a.npair = a.paired ? (a.nblk + 1) / 2 : a.nblk;
  a.ngrp = hq / (hpw * hgw);
  a.nwg = a.npair * a.ngrp * batch;
  dim3 grid(a.nwg);
  const bool bf = dtype == YR_DTYPE_BF16;
#define YR_PF(H, W)                                                                                        \
  if (hpw == H && hgw == W) {                                                                              \
    if (bf) hipLaunchKernelGGL((gqa_prefill_kernel<DT_BF16, H, W>), grid, dim3(256 * W), 0, st, a);         \
    else hipLaunchKernelGGL((gqa_prefill_kernel<DT_F16, H, W>), grid, dim3(256 * W), 0, st, a);             \
  }
  YR_PF(1, 1) YR_PF(1, 2) YR_PF(2, 1) YR_PF(2, 2)
#undef YR_PF
  YR_CHECK_LAUNCH(nm);
  return YR_OK;
}

// ---------------------------------------------------------------- no-allocation decode
// Device-resident scratch of yr_hip_gqa_decode_paged_noalloc: arrival
// tickets in [0, kTicketBytes), split records after them.  One copy per GPU,
// held until the process ends; every call on a GPU shares it, so calls that
// overlap on one GPU race.  Host code never passes `scratch` itself to a
// kernel (in host code the name is a stand-in, not a device address): it
// uses the address hipGetSymbolAddress returns for the current device.
// Its size covers every shape the decode accepts: the plan gives each of the
// B * Hkv (sequence, kv head) pairs ceil(DEC_TARGET_WG / pairs) splits or
// one (then no records), so records exist for fewer than 2 * DEC_TARGET_WG
// splits of at most 16 rows of D + 2 floats (D = 128).
constexpr size_t kNoAllocScratchBytes = kTicketBytes + (size_t)2 * DEC_TARGET_WG * 16 * (128 + 2) * sizeof(float);
static __device__ __align__(256) uint8_t scratch[kNoAllocScratchBytes];

constexpr int kMaxDevices = 64;
static void* g_scratch_ptr[kMaxDevices];
static std::mutex g_scratch_mu;

__global__ void fill_u32_kernel(uint32_t* p, int n, uint32_t v) {
  for (int i = blockIdx.x * blockDim.x + threadIdx.x; i < n; i += gridDim.x * blockDim.x) p[i] = v;
}

// Device address of this device's scratch (looked up once per device, with
// that device current).
static int noalloc_scratch(const char* nm, void** out) {
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return check_hip(e, nm);
  if (dev < 0 || dev >= kMaxDevices) return fail(YR_E_INVALID, "%s: device %d out of range", nm, dev);
  std::lock_guard<std::mutex> lk(g_scratch_mu);
  if (!g_scratch_ptr[dev]) {
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !p) return fail(YR_E_HIP, "%s: hipGetSymbolAddress(scratch) failed (%d)", nm, (int)e);
    g_scratch_ptr[dev] = p;
  }
  *out = g_scratch_ptr[dev];
  return YR_OK;
}

extern "C" {

size_t yr_hip_gqa_decode_noalloc_max_bytes(void) { return kNoAllocScratchBytes; }

int yr_hip_gqa_decode_paged(const void* q, const void* k_cache, const void* v_cache, const int32_t* kv_indptr,
                            const int32_t* kv_indices, const int32_t* kv_len, void* out, int batch, int hq,
                            int hkv, int d, int page_size, int max_kv_len, int dtype, void* workspace,
                            size_t workspace_bytes, void* stream) {
  return gqa_decode_launch("yr_hip_gqa_decode_paged", q, k_cache, v_cache, kv_indptr, kv_indices, kv_len, out, batch,
                           hq, hkv, d, page_size, max_kv_len, dtype, workspace, workspace_bytes, (hipStream_t)stream,
                           1.f / sqrtf((float)d));
}

int yr_hip_gqa_decode_paged_noalloc(const void* q, const void* k_cache, const void* v_cache,
                                    const int32_t* kv_indptr, const int32_t* kv_indices, const int32_t* kv_len,
                                    void* out, int batch, int hq, int hkv, int d, int page_size, int max_kv_len,
                                    int dtype, void* stream) {
  const char* nm = "yr_hip_gqa_decode_paged_noalloc";
  // every check before the ticket fill, so a rejected call launches nothing
  int rc = gqa_decode_check(nm, q, k_cache, v_cache, kv_indptr, kv_indices, kv_len, out, batch, hq, hkv, d,
                            page_size, max_kv_len, dtype);
  if (rc != YR_OK) return rc;
  const size_t need = yr_hip_gqa_decode_workspace(batch, hq, hkv, d, max_kv_len, page_size);
  if (need > kNoAllocScratchBytes)
    return fail(YR_E_WORKSPACE, "%s: needs %zu bytes of scratch, above the fixed %zu", nm, need,
                kNoAllocScratchBytes);
  void* ws = nullptr;
  rc = noalloc_scratch(nm, &ws);
  if (rc != YR_OK) return rc;
  hipStream_t st = (hipStream_t)stream;
  if (need) {
    // the tickets this call uses start at zero whatever an earlier call left
    // (a fill kernel, not a memset node, so the call can be graph-captured)
    const int nt = batch * hkv;
    hipLaunchKernelGGL(fill_u32_kernel, dim3((nt + 255) / 256), dim3(256), 0, st, (uint32_t*)ws, nt, 0u);
    YR_CHECK_LAUNCH(nm);
  }
  return gqa_decode_launch(nm, q, k_cache, v_cache, kv_indptr, kv_indices, kv_len, out, batch, hq, hkv, d,
                           page_size, max_kv_len, dtype, need ? ws : nullptr, need ? kNoAllocScratchBytes : 0, st,
                           1.f / sqrtf((float)d));
}

int yr_hip_gqa_prefill(const void* q, const void* k, const void* v, void* out, int batch, int seq, int hq,
                       int hkv, int d, int causal, int dtype, void* stream) {
  if (seq <= 0 || hkv <= 0) return fail(YR_E_INVALID, "yr_hip_gqa_prefill: bad shape");
  const long long qld = (long long)hq * d, kld = (long long)hkv * d;
  return prefill_launch("yr_hip_gqa_prefill", q, k, v, out, batch, seq, seq, hq, hkv, d, causal, dtype, seq * qld,
                        (int)qld, seq * kld, (int)kld, seq * qld, (int)qld, 1.f / sqrtf((float)d),
                        (hipStream_t)stream);
}

int yr_hip_argmax(const void* x, int64_t* out, int rows, int n, int n_valid, int dtype, void* stream) {
  const char* nm = "yr_hip_argmax";
  if (!x || !out) return fail(YR_E_INVALID, "%s: null pointer", nm);
  if (rows <= 0 || n <= 0 || n_valid <= 0 || n_valid > n) return fail(YR_E_INVALID, "%s: bad shape", nm);
  hipStream_t st = (hipStream_t)stream;
  if (dtype == YR_DTYPE_F16)
    hipLaunchKernelGGL(argmax_kernel<DT_F16>, dim3(rows), dim3(256), 0, st, (const uint16_t*)x, out, n, n_valid);
  else if (dtype == YR_DTYPE_BF16)
    hipLaunchKernelGGL(argmax_kernel<DT_BF16>, dim3(rows), dim3(256), 0, st, (const uint16_t*)x, out, n, n_valid);
  else
    return fail(YR_E_INVALID, "%s: dtype", nm);
  YR_CHECK_LAUNCH(nm);
  return YR_OK;
}

#ifdef YR_DEC_PROF
int yr_dec_prof_read(void* host) {
  return hipMemcpyFromSymbol(host, HIP_SYMBOL(yr::g_dec_prof), sizeof(yr::g_dec_prof)) == hipSuccess ? 0 : -1;
}
#endif

}  // extern "C"
