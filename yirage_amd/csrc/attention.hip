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
#include "yr_common.h"

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

// D = 128, G <= 16
template <int DT, int G>
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
  auto issue = [&](Blk& bk, int blk) __attribute__((always_inline)) {
    const int tb = c0 + blk * DEC_BLK;
#pragma unroll
    for (int n = 0; n < 2; n++) {
      const size_t off = tok_off(tb + 16 * n + lane % 16) + (lane / 16) * 8;
#pragma unroll
      for (int s = 0; s < 4; s++) bk.k[n][s] = ldg16(a.kc + off + 32 * s);
    }
#pragma unroll
    for (int i = 0; i < 8; i++) bk.v[i] = ldg16(a.vc + tok_off(tb + lane / 16 + 4 * i) + (lane % 16) * 8);
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
constexpr int PF_WAVES = 4;
constexpr int PF_THREADS = PF_WAVES * kWave;
constexpr int PF_QROWS = 16 * PF_WAVES;  // 64 query rows per workgroup
constexpr int PF_KT = 64;                // kv tokens per tile

struct PrefillArgs {
  const uint16_t* q;  // [B][S][Hq][D]
  const uint16_t* k;  // [B][S][Hkv][D]
  const uint16_t* v;
  uint16_t* o;
  int B, S, Hq, Hkv, causal;
  float scale_log2;
};

template <int DT>
__global__ __launch_bounds__(PF_THREADS) void gqa_prefill_kernel(PrefillArgs a) {
  constexpr int D = 128;
  // LDS: K tile [64 tok][128 d] (row pad 8 elems), V^T tile [128 d][64 tok] (pad 8)
  constexpr int KP = D + 8, VP = PF_KT + 8;
  __shared__ __align__(16) uint16_t sk[PF_KT * KP];
  __shared__ __align__(16) uint16_t svt[D * VP];
  __shared__ __align__(16) uint16_t sp[PF_WAVES][16 * (PF_KT + 8)];

  const int qt = blockIdx.x, h = blockIdx.y, b = blockIdx.z;
  const int G = a.Hq / a.Hkv, hk = h / G;
  const int tid = threadIdx.x, wave = tid / kWave, lane = tid % kWave;
  const int q0 = qt * PF_QROWS + wave * 16;  // first query row of this wave
  const size_t qstride = (size_t)a.Hq * D, kstride = (size_t)a.Hkv * D;

  // Q fragments (A operand): row q0 + lane%16, d = 32 s + 8 (lane/16)
  uint4 qf[4];
  {
    int r = q0 + lane % 16;
    const uint16_t* qrow = a.q + ((size_t)b * a.S + r) * qstride + (size_t)h * D;
#pragma unroll
    for (int s = 0; s < 4; s++)
      qf[s] = r < a.S ? ldg16(qrow + 32 * s + (lane / 16) * 8) : make_uint4(0, 0, 0, 0);
  }
  f32x4 acc[8];  // O[16 rows][128 d] as 8 n-tiles of 16 d
#pragma unroll
  for (int n = 0; n < 8; n++) acc[n] = f32x4{0.f, 0.f, 0.f, 0.f};
  float m_i[4], l_i[4];  // rows 4*(lane/16)+i of the wave's 16
#pragma unroll
  for (int i = 0; i < 4; i++) {
    m_i[i] = -INFINITY;
    l_i[i] = 0.f;
  }

  const int wg_last_row = (qt + 1) * PF_QROWS - 1;
  const int kv_end = a.causal ? min(a.S, wg_last_row + 1) : a.S;
  for (int t0 = 0; t0 < kv_end; t0 += PF_KT) {
    __syncthreads();
    // stage K tile (row-major) and V tile (transposed) : 64 tok x 128 d each
    for (int c = tid; c < PF_KT * (D / 8); c += PF_THREADS) {
      int tr = c / (D / 8), dc = (c % (D / 8)) * 8;
      int t = t0 + tr;
      uint4 kv = make_uint4(0, 0, 0, 0), vv = make_uint4(0, 0, 0, 0);
      if (t < a.S) {
        size_t off = ((size_t)b * a.S + t) * kstride + (size_t)hk * D + dc;
        kv = ldg16(a.k + off);
        vv = ldg16(a.v + off);
      }
      *reinterpret_cast<uint4*>(&sk[tr * KP + dc]) = kv;
      uint32_t vw[4] = {vv.x, vv.y, vv.z, vv.w};
#pragma unroll
      for (int e = 0; e < 4; e++) {
        svt[(dc + 2 * e) * VP + tr] = (uint16_t)(vw[e] & 0xffff);
        svt[(dc + 2 * e + 1) * VP + tr] = (uint16_t)(vw[e] >> 16);
      }
    }
    __syncthreads();
    if (a.causal && t0 > q0 + 15) continue;  // whole tile masked for this wave

    // S = Q K^T : 4 n-tiles of 16 tokens
    f32x4 s4[4];
#pragma unroll
    for (int j = 0; j < 4; j++) {
      f32x4 c = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int s = 0; s < 4; s++) {
        uint4 kb = *reinterpret_cast<const uint4*>(&sk[(16 * j + lane % 16) * KP + 32 * s + (lane / 16) * 8]);
        c = mfma16<DT>(qf[s], kb, c);
      }
      s4[j] = c;
    }
    // online softmax per row (row = 4*(lane/16)+i, col = token 16 j + lane%16)
#pragma unroll
    for (int i = 0; i < 4; i++) {
      int r = q0 + 4 * (lane / 16) + i;
      float mx = -INFINITY;
#pragma unroll
      for (int j = 0; j < 4; j++) {
        int t = t0 + 16 * j + lane % 16;
        bool ok = t < a.S && (!a.causal || t <= r);
        float v = ok ? s4[j][i] * a.scale_log2 : -INFINITY;
        s4[j][i] = v;
        mx = fmaxf(mx, v);
      }
#pragma unroll
      for (int o = 8; o > 0; o >>= 1) mx = fmaxf(mx, __shfl_xor(mx, o, kWave));
      float mnew = fmaxf(m_i[i], mx);
      float alpha = mnew == -INFINITY ? 1.f : exp2f(m_i[i] - mnew);
      float ls = 0.f;
#pragma unroll
      for (int j = 0; j < 4; j++) {
        float p = mnew == -INFINITY ? 0.f : exp2f(s4[j][i] - mnew);
        s4[j][i] = p;
        ls += p;
      }
#pragma unroll
      for (int o = 8; o > 0; o >>= 1) ls += __shfl_xor(ls, o, kWave);
      l_i[i] = l_i[i] * alpha + ls;
      m_i[i] = mnew;
#pragma unroll
      for (int n = 0; n < 8; n++) acc[n][i] *= alpha;
      // P (rounded to the input dtype) to LDS as [row][token]
#pragma unroll
      for (int j = 0; j < 4; j++)
        sp[wave][(4 * (lane / 16) + i) * (PF_KT + 8) + 16 * j + lane % 16] = (uint16_t)st_elem<DT>(s4[j][i]);
    }
    __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0): LDS writes of this wave done
    __builtin_amdgcn_wave_barrier();
    // O += P V : A = P[16 rows][32 tok] (lane: row lane%16, tok 8(lane/16)..), B = V[32 tok][16 d]
#pragma unroll
    for (int ks = 0; ks < 2; ks++) {
      uint4 pa = *reinterpret_cast<const uint4*>(&sp[wave][(lane % 16) * (PF_KT + 8) + 32 * ks + (lane / 16) * 8]);
#pragma unroll
      for (int n = 0; n < 8; n++) {
        uint4 vb = *reinterpret_cast<const uint4*>(&svt[(16 * n + lane % 16) * VP + 32 * ks + (lane / 16) * 8]);
        acc[n] = mfma16<DT>(pa, vb, acc[n]);
      }
    }
  }
  // write O rows 4*(lane/16)+i, d = 16 n + lane%16
#pragma unroll
  for (int i = 0; i < 4; i++) {
    int r = q0 + 4 * (lane / 16) + i;
    if (r >= a.S) continue;
    float inv = l_i[i] > 0.f ? 1.f / l_i[i] : 0.f;
    uint16_t* orow = a.o + ((size_t)b * a.S + r) * qstride + (size_t)h * D;
#pragma unroll
    for (int n = 0; n < 8; n++) orow[16 * n + lane % 16] = (uint16_t)st_elem<DT>(acc[n][i] * inv);
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

int yr_hip_gqa_decode_paged(const void* q, const void* k_cache, const void* v_cache, const int32_t* kv_indptr,
                            const int32_t* kv_indices, const int32_t* kv_len, void* out, int batch, int hq,
                            int hkv, int d, int page_size, int max_kv_len, int dtype, void* workspace,
                            size_t workspace_bytes, void* stream) {
  const char* nm = "yr_hip_gqa_decode_paged";
  if (!q || !k_cache || !v_cache || !kv_indptr || !kv_indices || !kv_len || !out)
    return fail(YR_E_INVALID, "%s: null pointer", nm);
  if (batch <= 0 || hkv <= 0 || hq % hkv) return fail(YR_E_INVALID, "%s: hq must be a multiple of hkv", nm);
  if (d != 128) return fail(YR_E_INVALID, "%s: head_dim %d unsupported (128)", nm, d);
  int G = hq / hkv;
  if (G != 1 && G != 2 && G != 4 && G != 8 && G != 16) return fail(YR_E_INVALID, "%s: group size %d", nm, G);
  if (page_size <= 0) return fail(YR_E_INVALID, "%s: bad page size", nm);
  if (dtype != YR_DTYPE_F16 && dtype != YR_DTYPE_BF16) return fail(YR_E_INVALID, "%s: dtype", nm);
  if (max_kv_len <= 0) return fail(YR_E_INVALID, "%s: max_kv_len must be > 0", nm);
  if (batch * hkv > kMaxTickets) return fail(YR_E_INVALID, "%s: batch * hkv too large", nm);
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
  if (dp.chunk / page_size + 2 > DEC_MAXPG)
    return fail(YR_E_INVALID, "%s: %d pages per split exceed %d (page_size too small)", nm, dp.chunk / page_size + 2,
                DEC_MAXPG);
  a.tickets = (uint32_t*)workspace;
  a.partial = need ? (float*)((char*)workspace + kTicketBytes) : nullptr;
  a.scale_log2 = kLog2e / sqrtf((float)d);
  dim3 grid(a.splits, hkv, batch);
  hipStream_t st = (hipStream_t)stream;
#define YR_DEC(G_)                                                                                        \
  if (G == G_) {                                                                                          \
    if (dtype == YR_DTYPE_F16) hipLaunchKernelGGL((gqa_decode_kernel<DT_F16, G_>), grid, dim3(DEC_THREADS), 0, st, a); \
    else hipLaunchKernelGGL((gqa_decode_kernel<DT_BF16, G_>), grid, dim3(DEC_THREADS), 0, st, a);         \
  }
  YR_DEC(1) YR_DEC(2) YR_DEC(4) YR_DEC(8) YR_DEC(16)
#undef YR_DEC
  YR_CHECK_LAUNCH(nm);
  return YR_OK;
}

int yr_hip_gqa_prefill(const void* q, const void* k, const void* v, void* out, int batch, int seq, int hq,
                       int hkv, int d, int causal, int dtype, void* stream) {
  const char* nm = "yr_hip_gqa_prefill";
  if (!q || !k || !v || !out) return fail(YR_E_INVALID, "%s: null pointer", nm);
  if (batch <= 0 || seq <= 0 || hkv <= 0 || hq % hkv) return fail(YR_E_INVALID, "%s: bad shape", nm);
  if (d != 128) return fail(YR_E_INVALID, "%s: head_dim %d unsupported (128)", nm, d);
  if (dtype != YR_DTYPE_F16 && dtype != YR_DTYPE_BF16) return fail(YR_E_INVALID, "%s: dtype", nm);
  PrefillArgs a;
  a.q = (const uint16_t*)q;
  a.k = (const uint16_t*)k;
  a.v = (const uint16_t*)v;
  a.o = (uint16_t*)out;
  a.B = batch;
  a.S = seq;
  a.Hq = hq;
  a.Hkv = hkv;
  a.causal = causal ? 1 : 0;
  a.scale_log2 = kLog2e / sqrtf((float)d);
  dim3 grid((seq + PF_QROWS - 1) / PF_QROWS, hq, batch);
  hipStream_t st = (hipStream_t)stream;
  if (dtype == YR_DTYPE_F16) hipLaunchKernelGGL(gqa_prefill_kernel<DT_F16>, grid, dim3(PF_THREADS), 0, st, a);
  else hipLaunchKernelGGL(gqa_prefill_kernel<DT_BF16>, grid, dim3(PF_THREADS), 0, st, a);
  YR_CHECK_LAUNCH(nm);
  return YR_OK;
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
