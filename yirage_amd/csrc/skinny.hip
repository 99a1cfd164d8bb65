// Skinny GEMMs with the weight in K x N layout (X[B][K] @ W[K][N], W row-major
// with columns contiguous) on MFMA for gfx950: RMSNorm+linear, gated MLP
// (SiLU(X W1) * (X W3)) and linear(+residual).
//
// The MFMA B operand wants eight consecutive k of one column per lane, the
// transpose of how W sits in memory.  Weight tiles therefore go to LDS
// unchanged (rows of 16 columns) and come back through ds_read_b64_tr_b16:
// within a 16-lane group, lane i element e of the result is element i % 4 of
// the 64-bit row that lane 4e + i / 4 addressed.  Lane j = 4e + q of group g
// addresses row 8g + e (+4 for the second read), columns 4q..4q+3, so lane i
// receives column i, rows 8g..8g+7: exactly its B fragment.
//
// Work split (stream-K): the (16-column tile, K chunk) units are dealt out in
// equal contiguous ranges to one persistent workgroup per CU.  A tile that
// straddles two ranges is finished by the last of its workgroups to arrive
// (arrival ticket; partial tiles as fp32 records, summed in workgroup order,
// so results do not depend on timing).  Workgroups are renumbered so that the
// four tiles sharing one 128-byte weight line run on one XCD (workgroup i runs
// on XCD i % 8): the line is fetched from HBM into that XCD's L2 once.
#include <type_traits>

#include "yr_common.h"

namespace yr {
namespace sk {

constexpr int kThreads = 512;
constexpr int kWaves = kThreads / kWave;
enum : int { EPI_LINEAR = 0, EPI_RMSNORM = 1, EPI_GATED = 2 };

struct Args {
  const uint16_t* x;         // [B][K]
  const uint16_t* gamma;     // [K] (RMSNorm) or null
  const uint16_t* w0;        // [K][N]
  const uint16_t* w1;        // [K][N] (gated: W3)
  const uint16_t* residual;  // [B][N] or null
  uint16_t* out;             // [B][N]
  float* partial;            // records of partial tiles: [workgroup][2][rec]
  uint32_t* tickets;         // [tiles], zero at rest
  int B, K, N;
  float eps;
  int kch;                   // K chunks (units) per tile
  int units;                 // tiles * kch
  int tw;                    // tile width in columns (batch-128 kernel)
};

// Unit range [lo(v), lo(v + 1)) of virtual workgroup v; the virtual workgroup
// that owns unit u.
__device__ __forceinline__ int unit_lo(int v, int U, int G) { return (int)(((long long)v * U) / G); }
__device__ __forceinline__ int owner_of(int u, int U, int G) { return (int)(((long long)(u + 1) * G - 1) / U); }


// 16-byte loads through a buffer descriptor: an offset at or past `bytes`
// returns zero without a memory access, so bounds checks need no branch (a
// branch per load would also make the compiler wait for every outstanding
// load where a count would do).
__device__ __forceinline__ __amdgpu_buffer_rsrc_t rsrc(const void* base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), 0, (int)bytes, 0x00020000);
}
__device__ __forceinline__ uint4 bload16(__amdgpu_buffer_rsrc_t r, uint32_t off) {
  return __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, 0));
}
constexpr uint32_t kOob = 0xfffffff0u;  // offset that is out of range for every buffer
constexpr int kSc1 = 16;                 // buffer cache policy: sc1 (agent-scope coherence)

// x * gamma, element-wise on 8 packed values, rounded to the storage type
// (the normalised activation the reference feeds its matmul)
template <int DT>
__device__ __forceinline__ uint4 scale8(uint4 x, uint4 g) {
  const uint32_t xv[4] = {x.x, x.y, x.z, x.w}, gv[4] = {g.x, g.y, g.z, g.w};
  uint32_t o[4];
#pragma unroll
  for (int i = 0; i < 4; i++)
    o[i] = pack2<DT>(lo16<DT>(xv[i]) * lo16<DT>(gv[i]), hi16<DT>(xv[i]) * hi16<DT>(gv[i]));
  return make_uint4(o[0], o[1], o[2], o[3]);
}

template <int DT>
__device__ __forceinline__ float sumsq8(uint4 x) {
  const uint32_t xv[4] = {x.x, x.y, x.z, x.w};
  float s = 0.f;
#pragma unroll
  for (int i = 0; i < 4; i++) {
    const float lo = lo16<DT>(xv[i]), hi = hi16<DT>(xv[i]);
    s += lo * lo + hi * hi;
  }
  return s;
}

// Epilogue of one output element from its full fp32 sums.
template <int DT, int EPI>
__device__ __forceinline__ void store_out(const Args& a, int b, int n, float v0, float v1, float ss) {
  float v = v0;
  if constexpr (EPI == EPI_RMSNORM) v *= rsqrtf(ss / (float)a.K + a.eps);
  else if constexpr (EPI == EPI_GATED) v = silu(v0) * v1;
  if (a.residual) v += ld_elem<DT>(a.residual[(size_t)b * a.N + n]);
  a.out[(size_t)b * a.N + n] = (uint16_t)st_elem<DT>(v);
}

// ---------------------------------------------------------------- B <= 16
// Tiles are TW columns wide (16, 32 or 64: NB = TW / 16 MFMA column blocks).
// Every wave streams its own share of the weights: a k step is 32 rows x TW
// columns of each matrix, NB 16-byte loads per lane per matrix (a load
// instruction covers 512 / TW rows of TW * 2 contiguous bytes), written to a
// wave-private LDS slot and read straight back as MFMA B fragments (LDS
// operations of one wave execute in order, so no barrier is involved).  A
// register ring keeps RING steps (weights, A fragment, gamma) in flight per
// wave, across unit and tile boundaries; only the end of a tile synchronises
// the workgroup, to add the waves' C tiles.
//
// Unit = KC rows of one tile; wave w takes steps [w SPW, (w+1) SPW) of every
// unit in its workgroup's range.
template <int DT, int NMAT, int EPI, int TW, int KC>
__global__ __launch_bounds__(kThreads, 1) void sk16_kernel(Args a) {
  constexpr int NB = TW / 16;                  // MFMA column blocks per tile
  constexpr int RPL = 512 / TW;                // rows per wave load instruction
  constexpr int SPW = KC / kWaves / 32;        // k steps per wave per unit
  constexpr int RING = NB * NMAT >= 8 ? 2 : NB * NMAT >= 4 ? 16 / (NB * NMAT) : 8;  // steps in flight (8-16 KiB per wave)
  constexpr bool NORM = EPI == EPI_RMSNORM;
  constexpr int CT = NMAT * 16 * TW;           // C tile floats (all matrices)
  constexpr int REC = CT + 16;                 // + row sums of squares
  static_assert(SPW >= 1 && KC % (kWaves * 32) == 0, "unit must give every wave whole k steps");
  // wave-private: one step; the next step's stores follow this step's reads
  // in the wave's in-order LDS queue
  __shared__ __attribute__((aligned(16))) uint16_t slot[kWaves][NMAT][32 * TW];
  __shared__ float red[kWaves][REC];
  __shared__ float fin[REC];

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int G = gridDim.x, U = a.units, KCH = a.kch;
  // XCD-grouped order when G % 8 == 0; the host launches G <= U workgroups,
  // so every range holds at least one unit
  const int v = G & 7 ? (int)blockIdx.x : (blockIdx.x & 7) * (G >> 3) + (blockIdx.x >> 3);
  const int ub = unit_lo(v, U, G), ue = unit_lo(v + 1, U, G);
  const int nsteps = (ue - ub) * SPW;  // this wave's steps

  const __amdgpu_buffer_rsrc_t rw0 = rsrc(a.w0, (uint32_t)((size_t)a.K * a.N * 2));
  const __amdgpu_buffer_rsrc_t rw1 = rsrc(NMAT == 2 ? a.w1 : a.w0, (uint32_t)((size_t)a.K * a.N * 2));
  const __amdgpu_buffer_rsrc_t rx = rsrc(a.x, (uint32_t)((size_t)a.B * a.K * 2));
  const __amdgpu_buffer_rsrc_t rg = rsrc(a.gamma, a.gamma ? (uint32_t)(a.K * 2) : 0u);
  const int arow = lane & 15;
  // weight load p of a step: lane -> row p RPL + lane / (TW / 8), columns 8 (lane % (TW / 8)) ..
  const int wrow = lane / (TW / 8), wcol = 8 * (lane % (TW / 8));

  struct Step {
    uint4 w[NMAT][NB];
    uint4 x;
    uint4 g;
  };
  // step i of this wave -> unit ub + i / SPW, rows k0 + 32 (wave SPW + i % SPW)
  auto issue = [&](Step& st, int i) __attribute__((always_inline)) {
    const int u = ub + i / SPW, t = u / KCH;
    const int kb = (u - t * KCH) * KC + 32 * (wave * SPW + i % SPW);  // first row of the step
    const bool ok = i < nsteps;
    const int n = t * TW + wcol;
#pragma unroll
    for (int p = 0; p < NB; p++) {
      const int kw = kb + p * RPL + wrow;
      const uint32_t woff = ok && kw < a.K && n < a.N ? (uint32_t)(((size_t)kw * a.N + n) * 2) : kOob;
      st.w[0][p] = bload16(rw0, woff);
      if constexpr (NMAT == 2) st.w[1][p] = bload16(rw1, woff);
    }
    const int kx = kb + 8 * (lane >> 4);
    st.x = bload16(rx, ok && kx < a.K && arow < a.B ? (uint32_t)(((size_t)arow * a.K + kx) * 2) : kOob);
    if constexpr (NORM) st.g = bload16(rg, ok && kx < a.K ? (uint32_t)(kx * 2) : kOob);
  };

  f32x4 acc[NMAT][NB];
#pragma unroll
  for (int m = 0; m < NMAT; m++)
#pragma unroll
    for (int q = 0; q < NB; q++) acc[m][q] = f32x4{0.f, 0.f, 0.f, 0.f};
  float ss = 0.f;  // this lane's sum of squares of x row lane % 16 (RMSNorm)

  // end of tile t within this workgroup's range: add the waves' C tiles (and
  // RMSNorm row sums of squares), then emit it or combine it across workgroups
  auto finish_tile = [&](int t) __attribute__((always_inline)) {
    // C block q of this wave: lane holds rows 4 (lane / 16) + i, column 16 q + lane % 16
#pragma unroll
    for (int m = 0; m < NMAT; m++)
#pragma unroll
      for (int q = 0; q < NB; q++)
#pragma unroll
        for (int i = 0; i < 4; i++)
          red[wave][m * 16 * TW + (4 * (lane >> 4) + i) * TW + 16 * q + (lane & 15)] = acc[m][q][i];
    if constexpr (NORM) {
      float s2 = ss + __shfl_xor(ss, 16, kWave);
      s2 += __shfl_xor(s2, 32, kWave);
      if (lane < 16) red[wave][CT + lane] = s2;
    }
    __syncthreads();
    for (int i = tid; i < REC; i += kThreads) {
      float sum = 0.f;
#pragma unroll
      for (int w = 0; w < kWaves; w++) sum += red[w][i];
      fin[i] = sum;
    }
    __syncthreads();
    const int tu0 = t * KCH, tu1 = tu0 + KCH;  // units of tile t
    const int n0 = t * TW;
    bool emit = true;
    if (tu0 < ub || tu1 > ue) {
      // partial tile: record slot (v, side), then the last contributor sums
      const int side = ub >= tu0 ? 0 : 1;  // 0: tile t is this range's first tile
      float* rec = a.partial + ((size_t)v * 2 + side) * REC;
      for (int i = tid * 4; i < REC; i += kThreads * 4)
        st_agent4(rec + i, make_float4(fin[i], fin[i + 1], fin[i + 2], fin[i + 3]));
      const int c0 = owner_of(tu0, U, G), c1 = owner_of(tu1 - 1, U, G);
      emit = arrive_last(&a.tickets[t], c1 - c0 + 1);
      if (emit) {
        // contributors' records in workgroup order, up to 8 loads in flight
        // per thread (a load consumed in the same loop iteration would cost
        // one memory round trip per contributor)
        // only the first contributor's range can start before the tile
        const int side0 = unit_lo(c0, U, G) >= tu0 ? 0 : 1;
        for (int i = tid * 4; i < REC; i += kThreads * 4) {
          float4 sum = make_float4(0.f, 0.f, 0.f, 0.f);
          for (int cb = c0; cb <= c1; cb += 8) {
            float4 r[8];
#pragma unroll
            for (int j = 0; j < 8; j++) {
              const int c = cb + j;
              const int cside = c == c0 ? side0 : 0;
              r[j] = c <= c1 ? ld_agent4(a.partial + ((size_t)c * 2 + cside) * REC + i) : make_float4(0.f, 0.f, 0.f, 0.f);
            }
#pragma unroll
            for (int j = 0; j < 8; j++)
              if (cb + j <= c1) {
                sum.x += r[j].x; sum.y += r[j].y; sum.z += r[j].z; sum.w += r[j].w;
              }
          }
          fin[i] = sum.x; fin[i + 1] = sum.y; fin[i + 2] = sum.z; fin[i + 3] = sum.w;
        }
        __syncthreads();
      }
    }
    if (emit) {
      for (int i = tid; i < a.B * TW; i += kThreads) {
        const int b = i / TW, col = i % TW, n = n0 + col;
        if (n < a.N)
          store_out<DT, EPI>(a, b, n, fin[b * TW + col], NMAT == 2 ? fin[16 * TW + b * TW + col] : 0.f,
                             NORM ? fin[CT + b] : 0.f);
      }
    }
#pragma unroll
    for (int m = 0; m < NMAT; m++)
#pragma unroll
      for (int q = 0; q < NB; q++) acc[m][q] = f32x4{0.f, 0.f, 0.f, 0.f};
    ss = 0.f;
    __syncthreads();  // red / fin are reused by the next tile
  };

  Step ring[RING];
#pragma unroll
  for (int j = 0; j < RING; j++) issue(ring[j], j);
  // consume step i from ring slot i % RING (compile-time within the unrolled
  // block), then put step i + RING in flight in the same registers.  Steps
  // past the end load zeros (out-of-range offsets), so the body runs without
  // a branch around its loads; only the tile end is conditional.
  for (int i0 = 0; i0 < nsteps; i0 += RING) {
#pragma unroll
    for (int j = 0; j < RING; j++) {
      const int i = i0 + j;
      Step& st = ring[j];
#pragma unroll
      for (int m = 0; m < NMAT; m++)
#pragma unroll
        for (int p = 0; p < NB; p++)
          *reinterpret_cast<uint4*>(slot[wave][m] + (p * RPL + wrow) * TW + wcol) = st.w[m][p];
      uint4 xa = st.x;
      if constexpr (NORM) {
        ss += sumsq8<DT>(xa);
        if (a.gamma) xa = scale8<DT>(xa, st.g);  // no gamma: x as is
      }
#pragma unroll
      for (int m = 0; m < NMAT; m++)
#pragma unroll
        for (int q = 0; q < NB; q++)
          acc[m][q] = mfma16<DT>(xa, b_frag(slot[wave][m] + 16 * q, TW, 0, lane), acc[m][q]);
      issue(st, i + RING);
      const int u = ub + i / SPW;
      if (i < nsteps && i % SPW == SPW - 1 && (u == ue - 1 || (u + 1) % KCH == 0)) finish_tile(u / KCH);
    }
  }
}

// ---------------------------------------------------------------- B <= 128
// A GEMM tile: all 128 rows x 64 columns of each matrix over one K split.
// Chunks of 64 K rows of W (64 x 64 per matrix) and x (128 x 64) go through
// registers (CHQ chunks in flight per thread) into a double-buffered LDS
// stage; wave w owns rows 32 (w % 4) .. +32 and columns 32 (w / 4) .. +32
// (2 x 2 MFMA blocks per matrix), A fragments by ds_read_b128, B fragments
// by transposing reads.  Splits of one tile add up through fp32 records and
// an arrival ticket (in split order).
// 64-column W rows (128 bytes) with their 16-byte chunks permuted by
// w_swz(row): the rows a transposing 32-lane read touches (8g + e and
// 8g + e + 4 for e < 4, g < 2) get distinct chunk pairs
__device__ __forceinline__ int w_swz(int r) { return (((r >> 1) & 1) | (((r >> 3) & 1) << 1)) << 1; }
// b_frag of a w_swz-permuted 64-column tile: 16 columns from chunk cb
__device__ __forceinline__ uint4 b_frag_swz(const uint16_t* tile, int cb, int row0, int lane) {
  const int g = lane >> 4, j = lane & 15, e = j >> 2, q = j & 3;
  const int r0 = row0 + 8 * g + e, r1 = r0 + 4, c = cb + (q >> 1);
  const uint16_t* p0 = tile + r0 * 64 + ((c ^ w_swz(r0)) << 3) + (q & 1) * 4;
  const uint16_t* p1 = tile + r1 * 64 + ((c ^ w_swz(r1)) << 3) + (q & 1) * 4;
  // an address-space cast (not an integer round trip) keeps the LDS object
  // visible to the compiler's wait analysis for direct-to-LDS loads
  auto cast = [](const uint16_t* p) __attribute__((always_inline)) {
    return (lds_v4i16*)(const_cast<uint16_t*>(p));
  };
  const uint2 l2 = __builtin_bit_cast(uint2, __builtin_amdgcn_ds_read_tr16_b64_v4i16(cast(p0)));
  const uint2 h2 = __builtin_bit_cast(uint2, __builtin_amdgcn_ds_read_tr16_b64_v4i16(cast(p1)));
  return make_uint4(l2.x, l2.y, h2.x, h2.y);
}

// 16 bytes per lane from a buffer straight into LDS (lane l's data lands at
// lds_block + 16 l, lds_block wave-uniform); an offset past the buffer
// writes zeros.  Issued as inline assembly: the compiler then inserts no
// waits of its own for these loads (it cannot tell which LDS stage one
// writes and would wait for all of them before any LDS read); the kernel
// orders them itself (s_waitcnt vmcnt + barrier before a stage is read, and
// a barrier after the last read of a stage before it is refilled).
typedef int yr_i32x4 __attribute__((ext_vector_type(4)));
__device__ __forceinline__ void bload_lds16(__amdgpu_buffer_rsrc_t r, uint32_t off, void* lds_block) {
  const uint32_t lds = __builtin_amdgcn_readfirstlane(
      (uint32_t)(uintptr_t)(__attribute__((address_space(3))) char*)(lds_block));
  asm volatile("s_mov_b32 m0, %1\n\tbuffer_load_dwordx4 %0, %2, 0 offen lds"
               :
               : "v"(off), "s"(lds), "s"(r)
               : "memory", "m0");
}

// s_waitcnt with only the vector-memory count constrained (gfx9 encoding:
// vmcnt bits 3:0 and 15:14, expcnt 6:4 and lgkmcnt 11:8 at their maxima)
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4) | (15 << 8));
}

// K-split partial sums of a batch-128 tile: every split stores its NV
// accumulator float4s in fragment order ([v][thread], one 1 KB store per
// wave and v) and, for RMSNorm, its 128 row sums of squares, then arrives on
// the tile's ticket; the last to arrive adds all records in split order (its
// own from registers) into acc / ssl and returns true, the others false.
// Records go through 128-bit loads / stores with the sc1 bit (the coherence
// of agent-scope atomics, but free to pipeline).  `active`: this thread
// holds accumulators.
template <int NV, bool NORM>
__device__ __forceinline__ bool merge_splits(const Args& a, int t, int splits, int sp, f32x4* acc, bool active,
                                             float* ssl) {
  constexpr int MB = 128;
  constexpr int REC = NV * kThreads * 4 + MB;  // floats
  const int tid = threadIdx.x;
  const __amdgpu_buffer_rsrc_t rp = rsrc(a.partial, (uint32_t)((size_t)a.units * REC * sizeof(float)));
  const uint32_t rec0 = (uint32_t)((size_t)t * splits * REC * sizeof(float));  // split 0 of this tile
  auto vrec = [&](int s2, int v) __attribute__((always_inline)) {
    return rec0 + (uint32_t)(((size_t)s2 * REC + ((size_t)v * kThreads + tid) * 4) * sizeof(float));
  };
  if (active) {
#pragma unroll
    for (int v = 0; v < NV; v++)
      __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(yr_u32x4, acc[v]), rp, vrec(sp, v), 0, kSc1);
  }
  const size_t ssoff = (size_t)t * splits * REC + NV * kThreads * 4;  // floats: split 0's row sums
  if (NORM && tid < MB) st_agent(a.partial + ssoff + (size_t)sp * REC + tid, ssl[tid]);
  if (!arrive_last(&a.tickets[t], splits)) return false;
  if (active) {
    // in groups of 8 float4s: sum = record 0 + record 1 + ..., in split order
#pragma unroll
    for (int v0 = 0; v0 < NV; v0 += 8) {
      constexpr int G = NV < 8 ? NV : 8;
      static_assert(NV % G == 0, "record groups");
      f32x4 sum[G];
#pragma unroll
      for (int v = 0; v < G; v++) sum[v] = f32x4{0.f, 0.f, 0.f, 0.f};
      for (int s2 = 0; s2 < splits; s2++) {
        f32x4 ld[G];
#pragma unroll
        for (int v = 0; v < G; v++)
          ld[v] = s2 == sp ? acc[v0 + v]
                           : __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(rp, vrec(s2, v0 + v), 0, kSc1));
#pragma unroll
        for (int v = 0; v < G; v++) sum[v] += ld[v];
      }
#pragma unroll
      for (int v = 0; v < G; v++) acc[v0 + v] = sum[v];
    }
  }
  if (NORM && tid < MB) {
    float ssum = 0.f;
    for (int s2 = 0; s2 < splits; s2++) ssum += ld_agent(a.partial + ssoff + (size_t)s2 * REC + tid);
    ssl[tid] = ssum;
  }
  __syncthreads();
  return true;
}

// NKL: W in N x K layout (W[N][K], torch Linear.weight).  Its rows already
// hold 8 consecutive k of one column per 16 bytes, the B fragment's order, so
// a W tile is staged like an x tile (64 padded rows of n) and B fragments
// come back by plain 16-byte reads.
template <int DT, int NMAT, int EPI, bool NKL>
__global__ __launch_bounds__(kThreads, 1) void sk128r_kernel(Args a) {
  constexpr int TW = 64, KS = 64, MB = 128;
  // K x N: W rows unpadded with chunks permuted by w_swz; x rows (and N x K
  // W rows) padded (fragments by 16-byte reads of 16 rows at one k)
  constexpr int LDX = KS + 8;
  constexpr int LDW = NKL ? LDX : TW;
  constexpr int WROWS = NKL ? TW : KS;
  static_assert(TW == 64, "w_swz / b_frag_swz assume 64-column W rows");
  constexpr int CHQ = 2;                      // chunks in flight (2 measured best of 2, 3, 4, 6)
  constexpr bool NORM = EPI == EPI_RMSNORM;
  __shared__ __attribute__((aligned(16))) uint16_t wl[2][NMAT][WROWS * LDW];
  __shared__ __attribute__((aligned(16))) uint16_t xl[2][MB * LDX];
  __shared__ float ssl[MB];

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int splits = a.kch;                   // K splits per tile
  const int t = blockIdx.x / splits, sp = blockIdx.x % splits;
  const int kper = (((a.K + splits - 1) / splits) + KS - 1) / KS * KS;  // rows per split (whole chunks)
  const int kbeg = sp * kper, kend = min(a.K, kbeg + kper);
  const int nchunks = kend > kbeg ? (kend - kbeg + KS - 1) / KS : 0;
  const int n0 = t * TW;

  const __amdgpu_buffer_rsrc_t rw0 = rsrc(a.w0, (uint32_t)((size_t)a.K * a.N * 2));
  const __amdgpu_buffer_rsrc_t rw1 = rsrc(NMAT == 2 ? a.w1 : a.w0, (uint32_t)((size_t)a.K * a.N * 2));
  const __amdgpu_buffer_rsrc_t rx = rsrc(a.x, (uint32_t)((size_t)a.B * a.K * 2));
  const __amdgpu_buffer_rsrc_t rg = rsrc(a.gamma, a.gamma ? (uint32_t)(a.K * 2) : 0u);
  // this thread's chunk pieces: W row tid / 8, columns 8 (tid % 8) (N x K:
  // column n0 + tid / 8, k 8 (tid % 8)); x rows tid / 8 and tid / 8 + 64,
  // k 8 (tid % 8)
  const int wr_ = tid >> 3, wc = 8 * (tid & 7);
  const int xr0 = tid >> 3, xk = 8 * (tid & 7);

  struct Chunk {
    uint4 w[NMAT];
    uint4 x[2];
    uint4 g;
  };
  auto issue = [&](Chunk& c, int ci) __attribute__((always_inline)) {
    const int k0 = kbeg + ci * KS;
    const bool ok = ci < nchunks;
    uint32_t woff;
    if constexpr (NKL) {
      const int n = n0 + wr_, kw = k0 + wc;
      woff = ok && kw < kend && n < a.N ? (uint32_t)(((size_t)n * a.K + kw) * 2) : kOob;
    } else {
      const int kw = k0 + wr_, n = n0 + wc;
      woff = ok && kw < kend && n < a.N ? (uint32_t)(((size_t)kw * a.N + n) * 2) : kOob;
    }
    c.w[0] = bload16(rw0, woff);
    if constexpr (NMAT == 2) c.w[1] = bload16(rw1, woff);
    const int kx = k0 + xk;
#pragma unroll
    for (int h = 0; h < 2; h++) {
      const int r = xr0 + 64 * h;
      c.x[h] = bload16(rx, ok && kx < kend && r < a.B ? (uint32_t)(((size_t)r * a.K + kx) * 2) : kOob);
    }
    if constexpr (NORM) c.g = bload16(rg, ok && kx < kend ? (uint32_t)(kx * 2) : kOob);
  };

  f32x4 acc[NMAT][2][2];
#pragma unroll
  for (int m = 0; m < NMAT; m++)
#pragma unroll
    for (int i = 0; i < 2; i++)
#pragma unroll
      for (int j = 0; j < 2; j++) acc[m][i][j] = f32x4{0.f, 0.f, 0.f, 0.f};
  float ss0 = 0.f, ss1 = 0.f;  // RMSNorm: sums of squares of x rows xr0, xr0 + 64 (this thread's k)
  const int mg = wave & 3, ng = wave >> 2;

  Chunk ring[CHQ];
#pragma unroll
  for (int j = 0; j < CHQ; j++) issue(ring[j], j);
  for (int c0 = 0; c0 < nchunks; c0 += CHQ) {
#pragma unroll
    for (int j = 0; j < CHQ; j++) {
      const int ci = c0 + j, lb = ci & 1;  // LDS stages alternate per chunk
      Chunk& c = ring[j];
      // stage chunk ci (x scaled by gamma for RMSNorm, row sums first)
#pragma unroll
      for (int m = 0; m < NMAT; m++)
        *reinterpret_cast<uint4*>(&wl[lb][m][wr_ * LDW + (NKL ? wc : ((wc >> 3) ^ w_swz(wr_)) << 3)]) = c.w[m];
#pragma unroll
      for (int h = 0; h < 2; h++) {
        uint4 xv = c.x[h];
        if constexpr (NORM) {
          (h ? ss1 : ss0) += sumsq8<DT>(xv);
          if (a.gamma) xv = scale8<DT>(xv, c.g);
        }
        *reinterpret_cast<uint4*>(&xl[lb][(xr0 + 64 * h) * LDX + xk]) = xv;
      }
      __syncthreads();
      issue(c, ci + CHQ);
#pragma unroll
      for (int ks = 0; ks < KS / 32; ks++) {
        uint4 af[2];
#pragma unroll
        for (int i = 0; i < 2; i++)
          af[i] = *reinterpret_cast<const uint4*>(&xl[lb][(32 * mg + 16 * i + (lane & 15)) * LDX + 32 * ks + 8 * (lane >> 4)]);
#pragma unroll
        for (int m = 0; m < NMAT; m++)
#pragma unroll
          for (int j2 = 0; j2 < 2; j2++) {
            const uint4 bf =
                NKL ? *reinterpret_cast<const uint4*>(
                          &wl[lb][m][(32 * ng + 16 * j2 + (lane & 15)) * LDW + 32 * ks + 8 * (lane >> 4)])
                    : b_frag_swz(wl[lb][m], 4 * ng + 2 * j2, 32 * ks, lane);
#pragma unroll
            for (int i = 0; i < 2; i++) acc[m][i][j2] = mfma16<DT>(af[i], bf, acc[m][i][j2]);
          }
      }
    }
  }
  // per-row sums of squares of this split (the 8 threads of a row are lanes
  // 8 r .. 8 r + 7 of one wave)
  if constexpr (NORM) {
#pragma unroll
    for (int o = 4; o > 0; o >>= 1) {
      ss0 += __shfl_xor(ss0, o, kWave);
      ss1 += __shfl_xor(ss1, o, kWave);
    }
    if ((tid & 7) == 0) {
      ssl[xr0] = ss0;
      ssl[xr0 + 64] = ss1;
    }
  }
  __syncthreads();
  // C element (matrix m, block i, j2, reg q) of this lane: row 32 mg + 16 i +
  // 4 (lane / 16) + q, column 32 ng + 16 j2 + lane % 16
  if (splits > 1 && !merge_splits<NMAT * 4, NORM>(a, t, splits, sp, &acc[0][0][0], true, ssl)) return;
#pragma unroll
  for (int i = 0; i < 2; i++)
#pragma unroll
    for (int j2 = 0; j2 < 2; j2++)
#pragma unroll
      for (int q = 0; q < 4; q++) {
        const int b = 32 * mg + 16 * i + 4 * (lane >> 4) + q, n = n0 + 32 * ng + 16 * j2 + (lane & 15);
        if (b < a.B && n < a.N)
          store_out<DT, EPI>(a, b, n, acc[0][i][j2][q], NMAT == 2 ? acc[NMAT - 1][i][j2][q] : 0.f,
                             NORM ? ssl[b] : 0.f);
      }
}

// Batches of 17..128 rows: one workgroup per (tile, K split), a tile TW
// columns of the output (128 when N allows >= 192 workgroups with two K
// splits, else 64), a K step ("chunk") 64 rows of W per matrix and the
// matching 128 x 64 block of x (whole 128-byte lines of x and of N x K W
// rows: half-line chunks fetch every line twice).
//
// The weight stream's rate is set by how wide a row segment each workgroup
// reads: with W in K x N layout the workgroups walk the rows of W in step,
// each taking TW columns of every row, and 256-byte segments stream ~12 %
// faster than 128-byte ones (measured on the gated-MLP weights, 2 x
// 4096 x 14336; 112-byte segments, 56-column tiles on all 256 CUs, are
// slower still).  Two K splits of 128-column tiles cost 1/16 extra bytes at
// K = 4096 in partial records, which the pair of workgroups of one tile (on
// one XCD) pass through that XCD's L2.
//
// Chunks arrive by direct buffer -> LDS loads (no registers), every 1 KB
// one load instruction, NST - 1 chunks ahead of the MFMAs.  Each wave waits
// for its own loads of a chunk (s_waitcnt vmcnt: one wave's loads complete
// in order) before the barrier that publishes it; a stage is refilled only
// after the barrier that follows its last read.  16-byte chunks of a row
// are permuted on the global side (the LDS image of one load instruction is
// contiguous) so that fragment reads are free of bank conflicts: 128-byte x
// rows (and N x K W rows) by row % 8, 128-byte K x N W rows by w_swz,
// 256-byte ones by w_swz256.
//
// NKL: W in N x K layout (W[N][K], torch Linear.weight).  Its rows already
// hold 8 consecutive k of one column per 16 bytes, the B fragment's order, so
// a W block is staged like an x block (TW rows of n) and B fragments come
// back by plain 16-byte reads.
__device__ __forceinline__ int x_swz(int r) { return r & 7; }
// chunk permutation of 256-byte rows: the rows one 32-lane transposing read
// touches (8g + e, and + 4, e < 4, g < 2) get distinct 32-byte chunk pairs
__device__ __forceinline__ int w_swz256(int r) { return ((r & 3) | (((r >> 3) & 1) << 2)) << 1; }
// b_frag of a w_swz256-permuted 128-column tile: 16 columns from chunk cb
__device__ __forceinline__ uint4 b_frag_swz256(const uint16_t* tile, int cb, int lane) {
  const int g = lane >> 4, j = lane & 15, e = j >> 2, q = j & 3;
  const int r0 = 8 * g + e, r1 = r0 + 4, c = cb + (q >> 1);
  const uint16_t* p0 = tile + r0 * 128 + ((c ^ w_swz256(r0)) << 3) + (q & 1) * 4;
  const uint16_t* p1 = tile + r1 * 128 + ((c ^ w_swz256(r1)) << 3) + (q & 1) * 4;
  auto cast = [](const uint16_t* p) __attribute__((always_inline)) {
    return (lds_v4i16*)(const_cast<uint16_t*>(p));
  };
  const uint2 l2 = __builtin_bit_cast(uint2, __builtin_amdgcn_ds_read_tr16_b64_v4i16(cast(p0)));
  const uint2 h2 = __builtin_bit_cast(uint2, __builtin_amdgcn_ds_read_tr16_b64_v4i16(cast(p1)));
  return make_uint4(l2.x, l2.y, h2.x, h2.y);
}

// s_waitcnt vmcnt(S * c) for a wave-uniform load count c (1 .. 8)
template <int S>
__device__ __forceinline__ void wait_loads(int c) {
  switch (c) {
    case 1: wait_vmcnt<S * 1>(); break;
    case 2: wait_vmcnt<S * 2>(); break;
    case 3: wait_vmcnt<S * 3>(); break;
    case 4: wait_vmcnt<S * 4>(); break;
    case 5: wait_vmcnt<S * 5>(); break;
    case 6: wait_vmcnt<S * 6>(); break;
    case 7: wait_vmcnt<S * 7>(); break;
    default: wait_vmcnt<S * 8>(); break;
  }
}

template <int DT, int NMAT, int EPI, bool NKL, int TW>
__global__ __launch_bounds__(kThreads, 1) void sk128_kernel(Args a) {
  constexpr int KS = 64, MB = 128;
  static_assert(EPI != EPI_RMSNORM, "RMSNorm runs in sk128r_kernel (x scaled on its way into LDS)");
  constexpr int WB = KS * TW * 2;              // bytes of one matrix's W chunk
  constexpr int XB = MB * KS * 2;              // bytes of one x chunk
  constexpr int SB = NMAT * WB + XB;           // bytes of a stage
  constexpr int NST = (144 * 1024) / SB;       // stages: 3 .. 6
  static_assert(NST >= 3, "LDS stages");
  constexpr int NBW = WB / 1024, NB = NMAT * NBW + XB / 1024;  // 1 KB load blocks per chunk
  constexpr int LMAX = (NB + kWaves - 1) / kWaves;
  // compute waves: each owns 64 rows x 32 columns (4 x 2 MFMA blocks: fewer
  // LDS fragment bytes per MFMA than 32 x 32) of every matrix, or with
  // SPLITM (two matrices, 64-column tiles) of one: waves 0-3 W1, 4-7 W3, so
  // that all eight waves compute; otherwise 64-column tiles leave waves 4-7
  // to loading
  constexpr bool SPLITM = NMAT == 2 && TW == 64;
  constexpr int MR = 4, NBC = 2, CW = SPLITM ? kWaves : 2 * TW / 32, NMW = SPLITM ? 1 : NMAT;
  static_assert(TW == 64 || TW == 128, "tile width");
  __shared__ __attribute__((aligned(16))) char stg[NST][SB];

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int splits = a.kch;  // K splits per tile
  // tiles (and the splits of one tile) of one XCD (workgroup i runs on XCD
  // i % 8) are contiguous: neighbours share DRAM pages, split pairs share L2
  const int bid = blockIdx.x;
  const int u = a.units % 8 == 0 ? (bid % 8) * (a.units / 8) + bid / 8 : bid;
  const int t = u / splits, sp = u % splits;
  const int kper = (((a.K + splits - 1) / splits) + KS - 1) / KS * KS;  // rows per split (whole chunks)
  const int kbeg = sp * kper, kend = min(a.K, kbeg + kper);
  const int nchunks = kend > kbeg ? (kend - kbeg + KS - 1) / KS : 0;
  const int n0 = t * TW, nlim = min(a.N, n0 + TW);

  const uint32_t wbytes = (uint32_t)((size_t)a.K * a.N * 2);
  const __amdgpu_buffer_rsrc_t rw0 = rsrc(a.w0, wbytes);
  const __amdgpu_buffer_rsrc_t rw1 = rsrc(NMAT == 2 ? a.w1 : a.w0, wbytes);
  const __amdgpu_buffer_rsrc_t rx = rsrc(a.x, (uint32_t)((size_t)a.B * a.K * 2));

  // load blocks j = wave + 8 i (i < cnt): j < NMAT NBW is W matrix j / NBW,
  // block j % NBW, else x block j - NMAT NBW.  Per block: byte offset at the
  // split's first chunk, the step per chunk, the k (relative to the chunk)
  // that must lie below kend (1 << 30: never), the offset into a stage.
  const int cnt = (NB - wave + kWaves - 1) / kWaves;
  uint32_t boff[LMAX], bstep[LMAX], bdst[LMAX];
  int bk[LMAX];
  __amdgpu_buffer_rsrc_t rs[LMAX];
#pragma unroll
  for (int i = 0; i < LMAX; i++) {
    const int j = wave + kWaves * i;
    bdst[i] = 1024u * (uint32_t)j;
    if (j < NMAT * NBW) {
      const int m = j / NBW, jb = j % NBW;
      rs[i] = m == 0 ? rw0 : rw1;
      if constexpr (NKL) {  // 8 rows (n) of 128 bytes (64 k)
        const int row = 8 * jb + (lane >> 3), src = (lane & 7) ^ x_swz(row), n = n0 + row;
        const bool ok = n < nlim;
        boff[i] = ok ? (uint32_t)(((size_t)n * a.K + kbeg + 8 * src) * 2) : kOob;
        bstep[i] = KS * 2;
        bk[i] = ok ? 8 * src : (1 << 30);
      } else {              // rows (k) of TW columns: 8 rows of 128 bytes or 4 of 256
        constexpr int CPR = TW / 8;
        const int row = (64 / CPR) * jb + lane / CPR, p = lane % CPR;
        const int src = p ^ (TW == 128 ? w_swz256(row) : w_swz(row)), n = n0 + 8 * src;
        const bool ok = n < nlim;
        boff[i] = ok ? (uint32_t)(((size_t)(kbeg + row) * a.N + n) * 2) : kOob;
        bstep[i] = (uint32_t)(KS * a.N * 2);
        bk[i] = ok ? row : (1 << 30);
      }
    } else {                // x: 8 rows of 128 bytes
      const int row = 8 * (j - NMAT * NBW) + (lane >> 3), src = (lane & 7) ^ x_swz(row);
      const bool ok = row < a.B && j < NB;
      rs[i] = rx;
      boff[i] = ok ? (uint32_t)(((size_t)row * a.K + kbeg + 8 * src) * 2) : kOob;
      bstep[i] = KS * 2;
      bk[i] = ok ? 8 * src : (1 << 30);
    }
  }

  auto issue = [&](int ci, int s) __attribute__((always_inline)) {
    const int krel = kend - kbeg - ci * KS;  // rows of the split left at chunk ci
#pragma unroll
    for (int i = 0; i < LMAX; i++) {
      if (i >= cnt) break;  // wave-uniform
      const uint32_t o = boff[i] + (uint32_t)ci * bstep[i];
      bload_lds16(rs[i], bk[i] < krel ? o : kOob, &stg[s][bdst[i]]);
    }
  };

  // compute wave w: rows 64 (w % 2) .., columns 32 (w / 2 % 2) .. of matrix
  // mw (SPLITM) or of every matrix
  const int mg = wave & 1, ng = (wave >> 1) & (TW / 32 - 1);
  const int mw = SPLITM ? wave >> 2 : 0;
  const bool cwave = wave < CW;
  f32x4 acc[NMW][MR][NBC];
#pragma unroll
  for (int m = 0; m < NMW; m++)
#pragma unroll
    for (int i = 0; i < MR; i++)
#pragma unroll
      for (int j = 0; j < NBC; j++) acc[m][i][j] = f32x4{0.f, 0.f, 0.f, 0.f};

  for (int ci = 0; ci < NST - 1; ci++) issue(ci, ci);
  int s = 0;  // stage of chunk ci
  for (int ci = 0; ci < nchunks; ci++) {
    // this wave's loads of chunk ci have landed (later chunks may be pending)
    wait_loads<NST - 2>(cnt);
    __syncthreads();
    issue(ci + NST - 1, s == 0 ? NST - 1 : s - 1);  // the stage chunk ci - 1 used
    const uint16_t* ws = reinterpret_cast<const uint16_t*>(&stg[s][0]);
    const uint16_t* xs = reinterpret_cast<const uint16_t*>(&stg[s][NMAT * WB]);
    if (cwave) {
#pragma unroll
      for (int ks = 0; ks < KS / 32; ks++) {
        const int lc = 4 * ks + (lane >> 4);
        uint4 af[MR];
#pragma unroll
        for (int i = 0; i < MR; i++) {
          const int r = 64 * mg + 16 * i + (lane & 15);
          af[i] = *reinterpret_cast<const uint4*>(&xs[r * KS + 8 * (lc ^ x_swz(r))]);
        }
#pragma unroll
        for (int m = 0; m < NMW; m++)
#pragma unroll
          for (int j2 = 0; j2 < NBC; j2++) {
            const uint16_t* wm = ws + (mw + m) * (WB / 2);
            uint4 bf;
            if constexpr (NKL) {
              const int r = 32 * ng + 16 * j2 + (lane & 15);
              bf = *reinterpret_cast<const uint4*>(&wm[r * KS + 8 * (lc ^ x_swz(r))]);
            } else if constexpr (TW == 128) {
              bf = b_frag_swz256(wm + 32 * ks * TW, 2 * (NBC * ng + j2), lane);
            } else {
              bf = b_frag_swz(wm, 2 * (NBC * ng + j2), 32 * ks, lane);
            }
#pragma unroll
            for (int i = 0; i < MR; i++) acc[m][i][j2] = mfma16<DT>(af[i], bf, acc[m][i][j2]);
          }
      }
    }
    s = s + 1 == NST ? 0 : s + 1;
  }
  wait_vm();  // loads past the last chunk (zeros into unused stages) have landed
  __syncthreads();
  // C element (block i, j2, reg q) of a compute lane: row 64 mg + 16 i +
  // 4 (lane / 16) + q, column 32 ng + 16 j2 + lane % 16
  if (splits > 1 && !merge_splits<NMW * MR * NBC, false>(a, t, splits, sp, &acc[0][0][0], cwave, nullptr)) return;
  // SPLITM: the W3 waves hand their sums to the W1 waves through LDS (the
  // stages are free: every load has landed and every wave is past its reads)
  f32x4 (*xch)[MR][NBC][kWave] = reinterpret_cast<f32x4 (*)[MR][NBC][kWave]>(&stg[0][0]);
  if constexpr (SPLITM) {
    static_assert(4 * MR * NBC * kWave * 16 <= NST * SB, "exchange fits the stages");
    if (mw == 1) {
#pragma unroll
      for (int i = 0; i < MR; i++)
#pragma unroll
        for (int j2 = 0; j2 < NBC; j2++) xch[wave - 4][i][j2][lane] = acc[0][i][j2];
    }
    __syncthreads();
    if (mw == 1) return;
  }
  if (!cwave) return;
#pragma unroll
  for (int i = 0; i < MR; i++)
#pragma unroll
    for (int j2 = 0; j2 < NBC; j2++) {
      const f32x4 v1 = SPLITM ? xch[wave][i][j2][lane] : acc[NMW - 1][i][j2];
#pragma unroll
      for (int q = 0; q < 4; q++) {
        const int b = 64 * mg + 16 * i + 4 * (lane >> 4) + q, n = n0 + 32 * ng + 16 * j2 + (lane & 15);
        if (b < a.B && n < nlim)
          store_out<DT, EPI>(a, b, n, acc[0][i][j2][q], NMAT == 2 ? v1[q] : 0.f, 0.f);
      }
    }
}

// ---------------------------------------------------------------- host side
constexpr int kGrid = 256;  // persistent workgroups (one per CU of an MI355X); a multiple of 8
constexpr int kTW = 64;     // tile width (columns)
constexpr int kKC = 1024;   // K rows per unit

struct Plan {
  int tw, kc, kch, units, tiles;
  size_t ws;
};

// 64-column tiles: every weight row segment a wave loads is one whole
// 128-byte line (narrower tiles leave the other parts of a line to other
// workgroups, which measured slower even with no cross-workgroup sums).
// Units of 1024 K rows, or 512 when only that deals every workgroup the
// same number of units (config 2a: 896 units of 1024 rows give workgroups 3
// or 4, 1792 of 512 give all 7; measured 45.2 -> 44.9 us).
inline Plan plan16(int K, int N, int nmat) {
  Plan p;
  p.tw = kTW;
  p.tiles = (N + p.tw - 1) / p.tw;
  const long long u1024 = (long long)p.tiles * ((K + kKC - 1) / kKC);
  const long long u512 = (long long)p.tiles * ((K + kKC / 2 - 1) / (kKC / 2));
  p.kc = u1024 % kGrid != 0 && u512 % kGrid == 0 ? kKC / 2 : kKC;
  p.kch = (K + p.kc - 1) / p.kc;
  p.units = p.tiles * p.kch;
  const int rec = nmat * 16 * kTW + 16;
  p.ws = kTicketBytes + (size_t)kGrid * 2 * rec * sizeof(float);
  return p;
}

}  // namespace sk
}  // namespace yr

namespace yr {

using namespace sk;

// Persistent grid: kGrid workgroups, fewer (a multiple of 8 when possible)
// when there are fewer units, so that no workgroup's range is empty.
static int grid_for(int units) { return units >= kGrid ? kGrid : units >= 8 ? units & ~7 : units; }

template <int DT, int NMAT, int EPI>
static void launch16(const Args& a, int kc, hipStream_t st) {
  const dim3 grid(grid_for(a.units)), block(kThreads);
  if (kc == kKC / 2) hipLaunchKernelGGL((sk16_kernel<DT, NMAT, EPI, kTW, kKC / 2>), grid, block, 0, st, a);
  else hipLaunchKernelGGL((sk16_kernel<DT, NMAT, EPI, kTW, kKC>), grid, block, 0, st, a);
}

// Batches of 17..128 rows run in sk128_kernel (direct-to-LDS) except
// RMSNorm (x is scaled on its way into LDS, which the direct loads skip) and
// the gated MLP with W in K x N layout, which run in sk128r_kernel
// (register-staged); measured on MI355X at B = 128, each is the faster of
// the two for its cases.
inline bool dma_path(int epi, bool nkl) { return epi != EPI_RMSNORM && !(epi == EPI_GATED && !nkl); }

// sk128_kernel: 128-column tiles with two K splits when that gives >= 192
// workgroups (N >= 12288), else 64-column tiles; sk128r_kernel: 64-column
// tiles.  K splits so that tiles x splits fills the CUs.
inline Plan plan128(int K, int N, int nmat, int epi, bool nkl) {
  Plan p;
  const bool dma = dma_path(epi, nkl);
  p.tw = dma && (N + 127) / 128 * 2 >= 192 ? 128 : 64;
  p.tiles = (N + p.tw - 1) / p.tw;
  int s = kGrid / p.tiles;
  const int maxs = (K + 63) / 64;
  s = s < 1 ? 1 : s > maxs ? maxs : s > 16 ? 16 : s;
  p.kch = s;
  p.kc = 0;
  p.units = p.tiles * s;
  // float4 accumulators per thread (merge_splits' NV): sk128_kernel 8 per
  // matrix a wave holds (one of two at 64 columns), sk128r_kernel 4 per matrix
  const int nv = dma ? (nmat == 2 && p.tw == 64 ? 1 : nmat) * 8 : nmat * 4;
  const size_t rec = (size_t)nv * kThreads * 4 + 128;  // floats
  p.ws = s > 1 ? kTicketBytes + (size_t)p.units * rec * sizeof(float) : 0;
  return p;
}

template <int DT, int NMAT, int EPI, bool NKL = false>
static void launch128(const Args& a, hipStream_t st) {
  if constexpr (EPI != EPI_RMSNORM && !(EPI == EPI_GATED && !NKL)) {  // dma_path
    if (a.tw == 128) hipLaunchKernelGGL((sk128_kernel<DT, NMAT, EPI, NKL, 128>), dim3(a.units), dim3(kThreads), 0, st, a);
    else hipLaunchKernelGGL((sk128_kernel<DT, NMAT, EPI, NKL, 64>), dim3(a.units), dim3(kThreads), 0, st, a);
  } else {
    hipLaunchKernelGGL((sk128r_kernel<DT, NMAT, EPI, NKL>), dim3(a.units), dim3(kThreads), 0, st, a);
  }
}

size_t skinny_kn_workspace(int B, int K, int N, int nmat, int epi) {
  size_t need = 0;
  for (int b0 = 0; b0 < B; b0 += 128) {
    const size_t w = B - b0 > 16 ? plan128(K, N, nmat, epi, false).ws : plan16(K, N, nmat).ws;
    if (w > need) need = w;
  }
  return need;
}

// X[B][K] @ W[K][N] (+ fused epilogue) for any B: passes of up to 128 rows
// (the batch-128 GEMM kernel above 16 rows, the skinny kernel below).
int skinny_kn(const uint16_t* x, const uint16_t* gamma, const uint16_t* w0, const uint16_t* w1,
              const uint16_t* residual, uint16_t* out, int B, int K, int N, float eps, int dtype, int nmat, int epi,
              void* ws, size_t ws_bytes, hipStream_t st, const char* name) {
  const size_t need = skinny_kn_workspace(B, K, N, nmat, epi);
  if (need > ws_bytes || (need && !ws))
    return fail(YR_E_WORKSPACE, "%s: workspace %zu < required %zu", name, ws_bytes, need);
  if ((N + 63) / 64 > kMaxTickets) return fail(YR_E_INVALID, "%s: N=%d too large", name, N);
  if ((size_t)K * N * 2 >= kOob || (size_t)B * K * 2 >= kOob)
    return fail(YR_E_INVALID, "%s: operands must be < 4 GiB (32-bit buffer offsets)", name);
  const bool bf = dtype == YR_DTYPE_BF16;
  for (int b0 = 0; b0 < B; b0 += 128) {
    const int rows = B - b0 < 128 ? B - b0 : 128;
    const bool big = rows > 16;
    const Plan p = big ? plan128(K, N, nmat, epi, false) : plan16(K, N, nmat);
    Args a = {};
    a.x = x + (size_t)b0 * K;
    a.gamma = gamma;
    a.w0 = w0;
    a.w1 = w1;
    a.residual = residual ? residual + (size_t)b0 * N : nullptr;
    a.out = out + (size_t)b0 * N;
    a.partial = (float*)((char*)ws + kTicketBytes);
    a.tickets = (uint32_t*)ws;
    a.B = rows;
    a.K = K;
    a.N = N;
    a.eps = eps;
    a.kch = p.kch;
    a.units = p.units;
    a.tw = p.tw;
#define YR_SK(DTV, NM, EP) (big ? launch128<DTV, NM, EP>(a, st) : launch16<DTV, NM, EP>(a, p.kc, st))
    if (nmat == 2) {
      if (bf) YR_SK(DT_BF16, 2, EPI_GATED); else YR_SK(DT_F16, 2, EPI_GATED);
    } else if (epi == EPI_RMSNORM) {
      if (bf) YR_SK(DT_BF16, 1, EPI_RMSNORM); else YR_SK(DT_F16, 1, EPI_RMSNORM);
    } else {
      if (bf) YR_SK(DT_BF16, 1, EPI_LINEAR); else YR_SK(DT_F16, 1, EPI_LINEAR);
    }
#undef YR_SK
    YR_CHECK_LAUNCH(name);
  }
  return YR_OK;
}

size_t skinny_nk128_workspace(int K, int N, int nmat, int epi) { return plan128(K, N, nmat, epi, true).ws; }

// One pass of 17..128 rows with W in N x K layout (the caller checked shapes,
// pointers and the workspace size).
int skinny_nk128(const uint16_t* x, const uint16_t* gamma, const uint16_t* w0, const uint16_t* w1,
                 const uint16_t* residual, uint16_t* out, int B, int K, int N, float eps, int dtype, int nmat,
                 int epi, void* ws, hipStream_t st, const char* name) {
  if ((N + 63) / 64 > kMaxTickets) return fail(YR_E_INVALID, "%s: N=%d too large", name, N);
  if ((size_t)K * N * 2 >= kOob || (size_t)B * K * 2 >= kOob)
    return fail(YR_E_INVALID, "%s: operands must be < 4 GiB (32-bit buffer offsets)", name);
  const Plan p = plan128(K, N, nmat, epi, true);
  Args a = {};
  a.x = x;
  a.gamma = gamma;
  a.w0 = w0;
  a.w1 = w1;
  a.residual = residual;
  a.out = out;
  a.partial = (float*)((char*)ws + kTicketBytes);
  a.tickets = (uint32_t*)ws;
  a.B = B;
  a.K = K;
  a.N = N;
  a.eps = eps;
  a.kch = p.kch;
  a.units = p.units;
  a.tw = p.tw;
  const bool bf = dtype == YR_DTYPE_BF16;
  if (nmat == 2) {
    if (bf) launch128<DT_BF16, 2, EPI_GATED, true>(a, st); else launch128<DT_F16, 2, EPI_GATED, true>(a, st);
  } else if (epi == EPI_RMSNORM) {
    if (bf) launch128<DT_BF16, 1, EPI_RMSNORM, true>(a, st); else launch128<DT_F16, 1, EPI_RMSNORM, true>(a, st);
  } else {
    if (bf) launch128<DT_BF16, 1, EPI_LINEAR, true>(a, st); else launch128<DT_F16, 1, EPI_LINEAR, true>(a, st);
  }
  YR_CHECK_LAUNCH(name);
  return YR_OK;
}

}  // namespace yr
