// Kernel-graph operators of the hip backend: the ops a KNGraph is built from
// (python/yirage/kernel.py:248-321; shape rules of src/kernel/matmul.cc,
// element_unary.cc, element_binary.cc, reduction.cc, rms_norm.cc), for the
// parts of a graph that no fused pattern covers, plus the kernel-graph form of
// attention (Q[G][M][d] x K^T[G][d][L] -> softmax -> x V[G][L][d]).
//
// Elementwise math is fp32 with one rounding to the 16-bit storage type per
// op, as the reference's transpiled element ops do
// (include/yirage/transpiler/runtime/kernel/element_unary.h:22-40,
// element_binary.h).  Every tensor handed to these kernels is dense
// row-major except where a stride list says otherwise.
#include <math.h>
#include <string.h>

#include <type_traits>

#include "attn_launch.h"
#include "yr_common.h"

namespace yr {
namespace graph {

// 32-bit unsigned division by a run-time constant, n < 2^31: q = (umulhi(n,
// m) + n) >> l with l = ceil(log2 d), m = floor(2^32 (2^l - d) / d) + 1
// (Granlund & Montgomery, "Division by invariant integers using
// multiplication", PLDI 1994, Figure 4.1).
struct FastDiv {
  uint32_t d, m, l;
};
static FastDiv fast_div(uint32_t d) {
  uint32_t l = 0;
  while ((1ull << l) < d) l++;
  const uint64_t m = ((1ull << 32) * ((1ull << l) - d)) / d + 1;
  return {d, (uint32_t)m, l};
}
__device__ __forceinline__ uint32_t fdiv(uint32_t n, const FastDiv& f) {
  return (__umulhi(n, f.m) + n) >> f.l;
}

// ------------------------------------------------------------------ pack
// dst[g][r][c] = c < C ? src[g s0 + r s1 + c s2] : 0 for c < Cd (destination
// strides d0 d1 d2).  One workgroup moves a 64 x 64 (r, c) tile through LDS:
// it reads along whichever of r / c is unit-stride in the source and writes
// along whichever is unit-stride in the destination, so transposing copies
// stay coalesced on both sides.
struct PackArgs {
  const uint16_t* src;
  uint16_t* dst;
  long long s0, s1, s2, d0, d1, d2;
  int R, C, Cd;  // rows, source columns, destination columns (>= C: zero padded)
  int src_c_unit, dst_c_unit;
};

__global__ __launch_bounds__(256) void pack_kernel(PackArgs a) {
  __shared__ uint16_t tile[64][66];
  const int g = blockIdx.z, r0 = blockIdx.y * 64, c0 = blockIdx.x * 64;
  const int t = threadIdx.x;
  const uint16_t* src = a.src + (size_t)g * a.s0;
#pragma unroll 4
  for (int i = 0; i < 16; i++) {
    const int u = t % 64, v = t / 64 + 4 * i;  // u runs along the unit-stride dim
    const int r = a.src_c_unit ? r0 + v : r0 + u;
    const int c = a.src_c_unit ? c0 + u : c0 + v;
    uint16_t x = 0;
    if (r < a.R && c < a.C) x = src[(size_t)r * a.s1 + (size_t)c * a.s2];
    tile[r - r0][c - c0] = x;
  }
  __syncthreads();
  uint16_t* dst = a.dst + (size_t)g * a.d0;
#pragma unroll 4
  for (int i = 0; i < 16; i++) {
    const int u = t % 64, v = t / 64 + 4 * i;
    const int r = a.dst_c_unit ? r0 + v : r0 + u;
    const int c = a.dst_c_unit ? c0 + u : c0 + v;
    if (r < a.R && c < a.Cd) dst[(size_t)r * a.d1 + (size_t)c * a.d2] = tile[r - r0][c - c0];
  }
}

static int pack(const char* nm, const void* src, void* dst, int G, int R, int C, int Cd, long long s0, long long s1,
                long long s2, long long d0, long long d1, long long d2, hipStream_t st) {
  PackArgs a;
  a.src = (const uint16_t*)src;
  a.dst = (uint16_t*)dst;
  a.s0 = s0; a.s1 = s1; a.s2 = s2; a.d0 = d0; a.d1 = d1; a.d2 = d2;
  a.R = R; a.C = C; a.Cd = Cd;
  a.src_c_unit = s2 == 1 || s1 != 1;
  a.dst_c_unit = d2 == 1 || d1 != 1;
  if (G <= 0 || R <= 0 || Cd <= 0 || G > 65535) return fail(YR_E_INVALID, "%s: pack shape", nm);
  dim3 grid((Cd + 63) / 64, (R + 63) / 64, G);
  if (grid.y > 65535) return fail(YR_E_INVALID, "%s: pack rows", nm);
  hipLaunchKernelGGL(pack_kernel, grid, dim3(256), 0, st, a);
  YR_CHECK_LAUNCH(nm);
  return YR_OK;
}

// ------------------------------------------------------------------ elementwise
enum UnaryKind { U_EXP = 0, U_SILU = 1, U_GELU = 2, U_RELU = 3, U_CLAMP = 4, U_SQRT = 5, U_SQUARE = 6, U_SCALE = 7 };
enum BinaryKind { B_ADD = 0, B_MUL = 1, B_DIV = 2, B_POW = 3 };

template <int DT>
__global__ __launch_bounds__(256) void unary_kernel(const uint16_t* x, uint16_t* y, long long n, int kind, float lo,
                                                    float hi) {
  for (long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (long long)gridDim.x * blockDim.x) {
    const float a = ld_elem<DT>(x[i]);
    float r;
    switch (kind) {
      case U_EXP: r = expf(a); break;
      case U_SILU: r = a / (1.f + expf(-a)); break;
      case U_GELU: r = 0.5f * a * (1.f + erff(a * 0.70710678118654752f)); break;
      case U_RELU: r = fmaxf(a, 0.f); break;
      case U_CLAMP: r = fminf(fmaxf(a, lo), hi); break;
      case U_SQRT: r = sqrtf(a); break;
      case U_SCALE: r = a * lo; break;
      default: r = a * a; break;
    }
    y[i] = (uint16_t)st_elem<DT>(r);
  }
}

constexpr int kMaxDims = 6;
struct BinaryArgs {
  const uint16_t* a;
  const uint16_t* b;
  uint16_t* out;
  long long n;
  int nd, kind;
  long long dims[kMaxDims];  // output dims
  long long sa[kMaxDims], sb[kMaxDims];  // element strides of a / b per output dim (0: broadcast)
  FastDiv div[kMaxDims];     // output dims as divisors (n < 2^31)
};

// Strided copy over up to 8 dims (16-bit elements): the tile gathers and
// scatters of a customized op run literally, one block tensor per tile
// tensor (src/kernel/customized.cc input / output maps).
constexpr int kCopyDims = 8;
struct CopyArgs {
  const uint16_t* src;
  uint16_t* dst;
  long long n;
  int nd;
  long long dims[kCopyDims], ss[kCopyDims], ds[kCopyDims];
};


// The same copy with collapsed dims and n < 2^31: division by multiplication.
struct CopyArgs32 {
  const uint16_t* src;
  uint16_t* dst;
  uint32_t n;
  int nd;
  FastDiv div[kCopyDims];
  long long ss[kCopyDims], ds[kCopyDims];
};

__global__ __launch_bounds__(256) void copy_nd32_kernel(CopyArgs32 p) {
  for (uint32_t i = blockIdx.x * blockDim.x + threadIdx.x; i < p.n; i += gridDim.x * blockDim.x) {
    uint32_t rem = i;
    long long os = 0, od = 0;
    for (int d = p.nd - 1; d >= 0; d--) {
      const uint32_t q = fdiv(rem, p.div[d]);
      const uint32_t c = rem - q * p.div[d].d;
      rem = q;
      os += (long long)c * p.ss[d];
      od += (long long)c * p.ds[d];
    }
    p.dst[od] = p.src[os];
  }
}

__global__ __launch_bounds__(256) void copy_nd_kernel(CopyArgs p) {
  for (long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x; i < p.n;
       i += (long long)gridDim.x * blockDim.x) {
    long long rem = i, os = 0, od = 0;
    for (int d = p.nd - 1; d >= 0; d--) {
      const long long c = rem % p.dims[d];
      rem /= p.dims[d];
      os += c * p.ss[d];
      od += c * p.ds[d];
    }
    p.dst[od] = p.src[os];
  }
}

template <int DT>
__global__ __launch_bounds__(256) void binary_kernel(BinaryArgs p) {
  for (long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x; i < p.n;
       i += (long long)gridDim.x * blockDim.x) {
    long long oa = 0, ob = 0;
    if (p.n < (1ll << 31)) {  // 32-bit index math, division by multiplication
      uint32_t rem = (uint32_t)i;
      for (int d = p.nd - 1; d >= 0; d--) {
        const uint32_t q = fdiv(rem, p.div[d]);
        const uint32_t c = rem - q * p.div[d].d;
        rem = q;
        oa += (long long)c * p.sa[d];
        ob += (long long)c * p.sb[d];
      }
    } else {
      long long rem = i;
      for (int d = p.nd - 1; d >= 0; d--) {
        const long long c = rem % p.dims[d];
        rem /= p.dims[d];
        oa += c * p.sa[d];
        ob += c * p.sb[d];
      }
    }
    const float x = ld_elem<DT>(p.a[oa]), y = ld_elem<DT>(p.b[ob]);
    float r;
    switch (p.kind) {
      case B_ADD: r = x + y; break;
      case B_MUL: r = x * y; break;
      case B_DIV: r = x / y; break;
      default: r = powf(x, y); break;
    }
    p.out[i] = (uint16_t)st_elem<DT>(r);
  }
}

// ------------------------------------------------------------------ fused elementwise
// A tree of unary / binary elementwise operators evaluated in one pass, one
// thread per output element: the fusion of single-consumer elementwise
// chains the reference's transpiler applies to threadblock graphs
// (src/transpiler/resolve_tb_fusion.cc:35-66), here over binary trees too.
// The program runs on a small register file; every operator's result is
// rounded to the element type, as the unfused chain stores it, so the
// output is bit-identical to running the operators one by one.
constexpr int kEwIn = 8, kEwProg = 32, kEwRegs = 16;
enum EwOp { EW_LOAD = 0, EW_UNARY = 1, EW_BINARY = 2 };
struct EwiseArgs {
  const uint16_t* in[kEwIn];
  uint16_t* out;
  uint32_t n;                    // < 2^31 (larger outputs are split by the host)
  int nd, nin, nprog;
  FastDiv div[kMaxDims];         // output dims
  uint32_t s[kEwIn][kMaxDims];   // element strides of each input per output dim (0: broadcast)
  int32_t op[kEwProg], dst[kEwProg], a[kEwProg], b[kEwProg], kind[kEwProg];  // dwords: scalar loads
  float lo[kEwProg], hi[kEwProg];
};

__device__ __forceinline__ float ew_unary(int kind, float a, float lo, float hi) {
  switch (kind) {
    case U_EXP: return expf(a);
    case U_SILU: return a / (1.f + expf(-a));
    case U_GELU: return 0.5f * a * (1.f + erff(a * 0.70710678118654752f));
    case U_RELU: return fmaxf(a, 0.f);
    case U_CLAMP: return fminf(fmaxf(a, lo), hi);
    case U_SQRT: return sqrtf(a);
    case U_SCALE: return a * lo;
    default: return a * a;
  }
}
__device__ __forceinline__ float ew_binary(int kind, float x, float y) {
  switch (kind) {
    case B_ADD: return x + y;
    case B_MUL: return x * y;
    case B_DIV: return x / y;
    default: return powf(x, y);
  }
}

// Each thread takes EPT elements (e, e + 256, ...), and the program is
// decoded once per instruction for all of them (its words are scalar loads
// whose latency would otherwise be paid per element).
template <int DT, int NR, int EPT>
__global__ __launch_bounds__(256) void ewise_kernel(EwiseArgs p) {
  for (uint32_t i0 = blockIdx.x * (256u * EPT) + threadIdx.x; i0 < p.n; i0 += gridDim.x * (256u * EPT)) {
    uint32_t c[EPT][kMaxDims];  // coordinates of the thread's elements
#pragma unroll
    for (int e = 0; e < EPT; e++) {
      uint32_t rem = i0 + 256u * e;
      if (rem >= p.n) rem = p.n - 1;  // (finite data for the lanes past the end; not stored)
#pragma unroll
      for (int d = kMaxDims - 1; d >= 0; d--) {
        if (d < p.nd) {
          const uint32_t q = fdiv(rem, p.div[d]);
          c[e][d] = rem - q * p.div[d].d;
          rem = q;
        } else {
          c[e][d] = 0;
        }
      }
    }
    // every input element first, all loads in flight at once (a load per
    // LOAD instruction would expose one memory latency per instruction)
    float lv[kEwIn][EPT];
#pragma unroll
    for (int q = 0; q < kEwIn; q++) {
      if (q < p.nin) {
#pragma unroll
        for (int e = 0; e < EPT; e++) {
          uint32_t o = 0;
#pragma unroll
          for (int d = 0; d < kMaxDims; d++) o += c[e][d] * p.s[q][d];
          lv[q][e] = ld_elem<DT>(p.in[q][o]);
        }
      } else {
#pragma unroll
        for (int e = 0; e < EPT; e++) lv[q][e] = 0.f;
      }
    }
    // registers are addressed with static indices only (a dynamically
    // indexed array would live in scratch memory)
    float r[NR][EPT];
#pragma unroll
    for (int k = 0; k < NR; k++)
#pragma unroll
      for (int e = 0; e < EPT; e++) r[k][e] = 0.f;
    float v[EPT];
    for (int j = 0; j < p.nprog; j++) {
      const int op = p.op[j], a = p.a[j], b = p.b[j], kind = p.kind[j], dst = p.dst[j];
      if (op == EW_LOAD) {
#pragma unroll
        for (int e = 0; e < EPT; e++) v[e] = lv[0][e];
#pragma unroll
        for (int q = 1; q < kEwIn; q++)
          if (a == q) {
#pragma unroll
            for (int e = 0; e < EPT; e++) v[e] = lv[q][e];
          }
      } else {
        float x[EPT], y[EPT];
#pragma unroll
        for (int e = 0; e < EPT; e++) { x[e] = r[0][e]; y[e] = r[0][e]; }
#pragma unroll
        for (int k = 1; k < NR; k++) {
          if (a == k) {
#pragma unroll
            for (int e = 0; e < EPT; e++) x[e] = r[k][e];
          }
          if (b == k) {
#pragma unroll
            for (int e = 0; e < EPT; e++) y[e] = r[k][e];
          }
        }
        if (op == EW_UNARY) {
          const float lo = p.lo[j], hi = p.hi[j];
#pragma unroll
          for (int e = 0; e < EPT; e++) v[e] = ld_elem<DT>((uint16_t)st_elem<DT>(ew_unary(kind, x[e], lo, hi)));
        } else {
#pragma unroll
          for (int e = 0; e < EPT; e++) v[e] = ld_elem<DT>((uint16_t)st_elem<DT>(ew_binary(kind, x[e], y[e])));
        }
      }
#pragma unroll
      for (int k = 0; k < NR; k++)
        if (dst == k) {
#pragma unroll
          for (int e = 0; e < EPT; e++) r[k][e] = v[e];
        }
    }
#pragma unroll
    for (int e = 0; e < EPT; e++)
      if (i0 + 256u * e < p.n) p.out[i0 + 256u * e] = (uint16_t)st_elem<DT>(v[e]);  // the last instruction's result
  }
}

// ------------------------------------------------------------------ reductions
// out[o][i] = sum_r x[o][r][i] (fp32) for long reductions: a workgroup takes
// one outer index and TX consecutive i (coalesced loads along i), its 256 /
// TX thread rows split r (thread row ty takes r = ty, ty + TY, ...), and the
// partial sums meet in LDS in thread-row order (deterministic).
template <int DT, bool MAX>
__global__ __launch_bounds__(256) void reduce_rows_kernel(const uint16_t* x, uint16_t* y, long long outer, int red,
                                                          long long inner, int lg_tx) {
  __shared__ float part[256];
  const int TX = 1 << lg_tx, TY = 256 >> lg_tx;
  const int tx = threadIdx.x & (TX - 1), ty = threadIdx.x >> lg_tx;
  const long long i = (long long)blockIdx.x * TX + tx;
  for (long long o = blockIdx.y; o < outer; o += gridDim.y) {
    float s = MAX ? -INFINITY : 0.f;
    if (i < inner) {
      const uint16_t* p = x + o * red * inner + i;
      for (int r = ty; r < red; r += TY) {
        const float v = ld_elem<DT>(p[(long long)r * inner]);
        s = MAX ? fmaxf(s, v) : s + v;
      }
    }
    part[threadIdx.x] = s;
    __syncthreads();
    if (ty == 0 && i < inner) {
      float t = part[tx];
      for (int k = 1; k < TY; k++) t = MAX ? fmaxf(t, part[k * TX + tx]) : t + part[k * TX + tx];
      y[o * inner + i] = (uint16_t)st_elem<DT>(t);
    }
    __syncthreads();
  }
}

// out[o][i] = sum_r x[o][r][i] (fp32), one thread per (o, i)
template <int DT, bool MAX = false>
__global__ __launch_bounds__(256) void reduce_kernel(const uint16_t* x, uint16_t* y, long long outer, int red,
                                                     long long inner) {
  const long long n = outer * inner;
  for (long long j = (long long)blockIdx.x * blockDim.x + threadIdx.x; j < n; j += (long long)gridDim.x * blockDim.x) {
    const long long o = j / inner, i = j % inner;
    const uint16_t* p = x + o * red * inner + i;
    float s = MAX ? -INFINITY : 0.f;
    for (int r = 0; r < red; r++) {
      const float v = ld_elem<DT>(p[(long long)r * inner]);
      s = MAX ? fmaxf(s, v) : s + v;
    }
    y[j] = (uint16_t)st_elem<DT>(s);
  }
}

// y[row] = x[row] * rsqrt(mean(x[row]^2) + eps): one workgroup per row
template <int DT>
__global__ __launch_bounds__(256) void rmsnorm_kernel(const uint16_t* x, uint16_t* y, int n, float eps) {
  const uint16_t* xr = x + (size_t)blockIdx.x * n;
  uint16_t* yr_ = y + (size_t)blockIdx.x * n;
  float ss = 0.f;
  for (int i = threadIdx.x; i < n; i += blockDim.x) {
    const float v = ld_elem<DT>(xr[i]);
    ss += v * v;
  }
  ss = wave_sum(ss);
  __shared__ float part[4];
  if (threadIdx.x % kWave == 0) part[threadIdx.x / kWave] = ss;
  __syncthreads();
  const float tot = part[0] + part[1] + part[2] + part[3];
  const float inv = rsqrtf(tot / (float)n + eps);
  for (int i = threadIdx.x; i < n; i += blockDim.x) yr_[i] = (uint16_t)st_elem<DT>(ld_elem<DT>(xr[i]) * inv);
}

// ------------------------------------------------------------------ batched matmul
// C[b] = A[b] (M x K, row-major) x B[b] (K x N, row-major), fp32 accumulate on
// MFMA 16x16x32.  Workgroup = 64 x 64 tile of C, 4 waves of 32 x 32 (2 x 2
// MFMA blocks); K in steps of 32 through LDS.  A fragments are 16-byte LDS
// reads of padded rows; B fragments come from the row-major K x N tile by
// transposing reads.  K and N must be multiples of 8 (16-byte rows).
constexpr int MM_T = 64, MM_KS = 32;
template <int DT>
__global__ __launch_bounds__(256) void matmul_kernel(const uint16_t* A, const uint16_t* B, uint16_t* C, int M, int N,
                                                     int K, long long sA, long long sB, long long sC) {
  constexpr int LDA = MM_KS + 8, LDB = MM_T + 8;
  __shared__ __attribute__((aligned(16))) uint16_t as[MM_T * LDA];
  __shared__ __attribute__((aligned(16))) uint16_t bs[MM_KS * LDB];
  const int b = blockIdx.z, m0 = blockIdx.y * MM_T, n0 = blockIdx.x * MM_T;
  const int t = threadIdx.x, lane = t % kWave, w = t / kWave;
  const int wm = (w / 2) * 32, wn = (w % 2) * 32;
  A += (size_t)b * sA;
  B += (size_t)b * sB;
  f32x4 acc[2][2];
#pragma unroll
  for (int i = 0; i < 2; i++)
#pragma unroll
    for (int j = 0; j < 2; j++) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};
  // staging: A tile 64 x 32 = 256 chunks of 8 (row t / 4, chunk t % 4);
  // B tile 32 x 64 = 256 chunks (row t / 8, chunk t % 8)
  const int ar = t / 4, ac = (t % 4) * 8, br = t / 8, bc = (t % 8) * 8;
  for (int k0 = 0; k0 < K; k0 += MM_KS) {
    uint4 av = make_uint4(0, 0, 0, 0), bv = make_uint4(0, 0, 0, 0);
    if (m0 + ar < M && k0 + ac < K) av = ldg16(A + (size_t)(m0 + ar) * K + k0 + ac);
    if (k0 + br < K && n0 + bc < N) bv = ldg16(B + (size_t)(k0 + br) * N + n0 + bc);
    __syncthreads();
    *reinterpret_cast<uint4*>(&as[ar * LDA + ac]) = av;
    *reinterpret_cast<uint4*>(&bs[br * LDB + bc]) = bv;
    __syncthreads();
    uint4 af[2], bf[2];
#pragma unroll
    for (int i = 0; i < 2; i++)
      af[i] = *reinterpret_cast<const uint4*>(&as[(wm + 16 * i + lane % 16) * LDA + (lane / 16) * 8]);
#pragma unroll
    for (int j = 0; j < 2; j++) bf[j] = b_frag(bs + wn + 16 * j, LDB, 0, lane);
#pragma unroll
    for (int i = 0; i < 2; i++)
#pragma unroll
      for (int j = 0; j < 2; j++) acc[i][j] = mfma16<DT>(af[i], bf[j], acc[i][j]);
  }
  C += (size_t)b * sC;
#pragma unroll
  for (int i = 0; i < 2; i++)
#pragma unroll
    for (int j = 0; j < 2; j++)
#pragma unroll
      for (int e = 0; e < 4; e++) {
        const int r = m0 + wm + 16 * i + 4 * (lane / 16) + e, c = n0 + wn + 16 * j + lane % 16;
        if (r < M && c < N) C[(size_t)r * N + c] = (uint16_t)st_elem<DT>(acc[i][j][e]);
      }
}

// identity page table of the kernel-graph decode: G sequences of L tokens,
// one page each
__global__ void page_iota_kernel(int32_t* indptr, int32_t* indices, int32_t* lens, int G, int L) {
  for (int i = blockIdx.x * blockDim.x + threadIdx.x; i <= G; i += gridDim.x * blockDim.x) {
    indptr[i] = i;
    if (i < G) {
      indices[i] = i;
      lens[i] = L;
    }
  }
}

// ------------------------------------------------------------------ graph attention
// O[g] = softmax(scale * Q[g] K[g]) V[g] with Q [G][M][d], K [G][d][L]
// (the kernel-graph operand: its rows are head dims), V [G][L][d], each given
// by three element strides.  Up to 16 query rows per group (a power of two)
// run on the split-KV decode kernel over an identity page table (one page of
// L tokens per group), more on the flash-attention prefill kernel.  Operands
// not already laid out as [G][rows][128] contiguous are packed into the
// workspace first (zero-padded to d = 128 for d < 128, which leaves the
// scores and the first d output columns unchanged).
struct AttnPlan {
  bool decode, pack_q, pack_k, pack_v, pack_o;
  size_t off_q, off_k, off_v, off_o, off_pt, dec_ws, total;
};

static bool dense_rows(const long long* s, int G, int rows, int d) {
  // [G][rows][d] contiguous with d == 128 (the group stride is unused when G == 1)
  return d == 128 && s[2] == 1 && s[1] == 128 && (G == 1 || s[0] == (long long)rows * 128);
}

static AttnPlan attn_plan(int G, int M, int L, int d, const long long* sq, const long long* sk, const long long* sv,
                          const long long* so) {
  AttnPlan p;
  // the decode kernel takes one arrival ticket per group (G <= kMaxTickets);
  // with one L-token page per group its page budget always fits
  p.decode = M <= 16 && (M & (M - 1)) == 0 && G <= kMaxTickets;
  p.pack_q = !dense_rows(sq, G, M, d);
  // K as the kernel wants it is [G][L][128]: K^T's strides swapped
  const long long skt[3] = {sk[0], sk[2], sk[1]};
  p.pack_k = !dense_rows(skt, G, L, d);
  p.pack_v = !dense_rows(sv, G, L, d);
  p.pack_o = !dense_rows(so, G, M, d);
  // the shared workspace layout: arrival tickets in [0, kTicketBytes) (zero
  // at rest, whichever operator ran last), then the decode's split records,
  // then the packed operands
  size_t off = kTicketBytes;
  auto take = [&](size_t bytes) {
    const size_t o = off;
    off += (bytes + 255) & ~(size_t)255;
    return o;
  };
  p.dec_ws = p.decode ? yr_hip_gqa_decode_workspace(G, M, 1, 128, L, L) : 0;
  if (p.dec_ws) take(p.dec_ws - kTicketBytes);
  p.off_q = p.pack_q ? take((size_t)G * M * 128 * 2) : 0;
  p.off_k = p.pack_k ? take((size_t)G * L * 128 * 2) : 0;
  p.off_v = p.pack_v ? take((size_t)G * L * 128 * 2) : 0;
  p.off_o = p.pack_o ? take((size_t)G * M * 128 * 2) : 0;
  p.off_pt = p.decode ? take((size_t)(3 * G + 1) * 4) : 0;
  p.total = off;
  return p;
}

}  // namespace graph
}  // namespace yr

using namespace yr;
using namespace yr::graph;

namespace {

int grid_for(long long n) {
  long long g = (n + 255) / 256;
  return (int)(g < 1 ? 1 : g > 8192 ? 8192 : g);
}

template <class F>
int by_dtype(int dtype, F f) {
  if (dtype == YR_DTYPE_F16) return f(std::integral_constant<int, DT_F16>{});
  if (dtype == YR_DTYPE_BF16) return f(std::integral_constant<int, DT_BF16>{});
  return fail(YR_E_INVALID, "graph op: dtype %d unsupported (f16 / bf16)", dtype);
}

// Short reductions (r <= 8, or enough outputs to fill the chip on their
// own) keep one thread per output; longer ones split r across a workgroup.
template <bool MAX>
int reduce_launch(const char* nm, const void* x, void* y, int64_t outer, int red, int64_t inner, int dtype,
                  hipStream_t st) {
  return by_dtype(dtype, [&](auto dt) {
    constexpr int D = decltype(dt)::value;
    if (red <= 8 || outer * inner >= (1 << 20)) {
      hipLaunchKernelGGL((reduce_kernel<D, MAX>), dim3(grid_for(outer * inner)), dim3(256), 0, st,
                         (const uint16_t*)x, (uint16_t*)y, (long long)outer, red, (long long)inner);
    } else {
      int lg = 0;
      while ((1 << lg) < inner && lg < 6) lg++;
      const long long gx = (inner + (1 << lg) - 1) >> lg;
      if (gx > 0x7fffffffLL) return fail(YR_E_INVALID, "%s: inner dim too large", nm);
      const unsigned gy = (unsigned)(outer < 65535 ? outer : 65535);
      hipLaunchKernelGGL((reduce_rows_kernel<D, MAX>), dim3((unsigned)gx, gy), dim3(256), 0, st, (const uint16_t*)x,
                         (uint16_t*)y, (long long)outer, red, (long long)inner, lg);
    }
    YR_CHECK_LAUNCH(nm);
    return YR_OK;
  });
}


}  // namespace

extern "C" {

size_t yr_hip_graph_attention_workspace(int G, int M, int L, int d, const int64_t* strides12) {
  if (G <= 0 || M <= 0 || L <= 0 || d <= 0 || d > 128 || !strides12) return 0;
  const long long* s = reinterpret_cast<const long long*>(strides12);
  return attn_plan(G, M, L, d, s, s + 3, s + 6, s + 9).total;
}

int yr_hip_graph_attention(const void* q, const void* k, const void* v, void* out, int G, int M, int L, int d,
                           const int64_t* strides12, float scale, int dtype, void* workspace, size_t workspace_bytes,
                           void* stream) {
  const char* nm = "yr_hip_graph_attention";
  if (!q || !k || !v || !out || !strides12) return fail(YR_E_INVALID, "%s: null pointer", nm);
  if (G <= 0 || M <= 0 || L <= 0 || d <= 0 || d > 128 || d % 8)
    return fail(YR_E_INVALID, "%s: shape G=%d M=%d L=%d d=%d (d <= 128, multiple of 8)", nm, G, M, L, d);
  if (dtype != YR_DTYPE_F16 && dtype != YR_DTYPE_BF16) return fail(YR_E_INVALID, "%s: dtype", nm);
  const long long* s = reinterpret_cast<const long long*>(strides12);
  const long long *sq = s, *sk = s + 3, *sv = s + 6, *so = s + 9;
  const AttnPlan p = attn_plan(G, M, L, d, sq, sk, sv, so);
  if (p.total > workspace_bytes || (p.total && !workspace))
    return fail(YR_E_WORKSPACE, "%s: workspace %zu < %zu", nm, workspace_bytes, p.total);
  hipStream_t st = (hipStream_t)stream;
  char* ws = (char*)workspace;
  const void* qd = q;
  const void* kd = k;
  const void* vd = v;
  void* od = out;
  int rc = YR_OK;
  const long long RM = (long long)M * 128, RL = (long long)L * 128;
  if (p.pack_q) {
    qd = ws + p.off_q;
    rc = pack(nm, q, ws + p.off_q, G, M, d, 128, sq[0], sq[1], sq[2], RM, 128, 1, st);
  }
  if (rc == YR_OK && p.pack_k) {  // rows of the packed K are tokens: source strides (g, token, dim)
    kd = ws + p.off_k;
    rc = pack(nm, k, ws + p.off_k, G, L, d, 128, sk[0], sk[2], sk[1], RL, 128, 1, st);
  }
  if (rc == YR_OK && p.pack_v) {
    vd = ws + p.off_v;
    rc = pack(nm, v, ws + p.off_v, G, L, d, 128, sv[0], sv[1], sv[2], RL, 128, 1, st);
  }
  if (rc != YR_OK) return rc;
  if (p.pack_o) od = ws + p.off_o;
  if (p.decode) {
    int32_t* pt = reinterpret_cast<int32_t*>(ws + p.off_pt);
    hipLaunchKernelGGL(page_iota_kernel, dim3((G + 256) / 256), dim3(256), 0, st, pt, pt + G + 1, pt + 2 * G + 1, G, L);
    YR_CHECK_LAUNCH(nm);
    rc = gqa_decode_launch(nm, qd, kd, vd, pt, pt + G + 1, pt + 2 * G + 1, od, G, M, 1, 128, L, L, dtype,
                           p.dec_ws ? ws : nullptr, p.dec_ws, st, scale);
  } else {
    rc = prefill_launch(nm, qd, kd, vd, od, G, M, L, 1, 1, 128, 0, dtype, RM, 128, RL, 128, RM, 128, scale, st);
  }
  if (rc == YR_OK && p.pack_o) rc = pack(nm, ws + p.off_o, out, G, M, d, d, RM, 128, 1, so[0], so[1], so[2], st);
  return rc;
}

int yr_hip_graph_pack(const void* src, void* dst, int g, int rows, int cols, int dst_cols, const int64_t* strides6,
                      int dtype, void* stream) {
  const char* nm = "yr_hip_graph_pack";
  if (!src || !dst || !strides6) return fail(YR_E_INVALID, "%s: null pointer", nm);
  if (dtype != YR_DTYPE_F16 && dtype != YR_DTYPE_BF16) return fail(YR_E_INVALID, "%s: dtype", nm);
  const long long* s = reinterpret_cast<const long long*>(strides6);
  return pack(nm, src, dst, g, rows, cols, dst_cols, s[0], s[1], s[2], s[3], s[4], s[5], (hipStream_t)stream);
}

int yr_hip_graph_copy_nd(const void* src, void* dst, int ndim, const int64_t* dims, const int64_t* src_strides,
                         const int64_t* dst_strides, int dtype, void* stream) {
  const char* nm = "yr_hip_graph_copy_nd";
  if (!src || !dst || !dims || !src_strides || !dst_strides) return fail(YR_E_INVALID, "%s: null pointer", nm);
  if (ndim <= 0 || ndim > kCopyDims) return fail(YR_E_INVALID, "%s: %d dims (1..%d)", nm, ndim, kCopyDims);
  if (dtype != YR_DTYPE_F16 && dtype != YR_DTYPE_BF16) return fail(YR_E_INVALID, "%s: dtype", nm);
  CopyArgs p;
  p.src = (const uint16_t*)src;
  p.dst = (uint16_t*)dst;
  p.nd = ndim;
  long long n = 1;
  for (int d = 0; d < ndim; d++) {
    if (dims[d] <= 0 || src_strides[d] < 0 || dst_strides[d] < 0)
      return fail(YR_E_INVALID, "%s: axis %d: dim %lld, strides %lld / %lld", nm, d, (long long)dims[d],
                  (long long)src_strides[d], (long long)dst_strides[d]);
    p.dims[d] = dims[d];
    p.ss[d] = src_strides[d];
    p.ds[d] = dst_strides[d];
    n *= dims[d];
  }
  p.n = n;
  hipStream_t st = (hipStream_t)stream;
  // collapse: drop unit dims, merge a dim into the next one when both
  // sides step through them contiguously
  long long cd[kCopyDims], cs[kCopyDims], cdst[kCopyDims];
  int m = 0;
  for (int d = 0; d < ndim; d++) {
    if (p.dims[d] == 1) continue;
    if (m > 0 && cs[m - 1] == p.ss[d] * p.dims[d] && cdst[m - 1] == p.ds[d] * p.dims[d]) {
      cd[m - 1] *= p.dims[d];
      cs[m - 1] = p.ss[d];
      cdst[m - 1] = p.ds[d];
      continue;
    }
    cd[m] = p.dims[d];
    cs[m] = p.ss[d];
    cdst[m] = p.ds[d];
    m++;
  }
  if (m == 0) {
    cd[0] = 1;
    cs[0] = cdst[0] = 0;
    m = 1;
  }
  if (n < (1ll << 31)) {
    CopyArgs32 q;
    q.src = p.src;
    q.dst = p.dst;
    q.n = (uint32_t)n;
    q.nd = m;
    for (int d = 0; d < m; d++) {
      q.div[d] = fast_div((uint32_t)cd[d]);
      q.ss[d] = cs[d];
      q.ds[d] = cdst[d];
    }
    hipLaunchKernelGGL(copy_nd32_kernel, dim3(grid_for(n)), dim3(256), 0, st, q);
  } else {
    hipLaunchKernelGGL(copy_nd_kernel, dim3(grid_for(n)), dim3(256), 0, st, p);
  }
  YR_CHECK_LAUNCH(nm);
  return YR_OK;
}

int yr_hip_graph_unary(const void* x, void* y, int64_t n, int kind, float lo, float hi, int dtype, void* stream) {
  const char* nm = "yr_hip_graph_unary";
  if (!x || !y || n <= 0) return fail(YR_E_INVALID, "%s: bad arguments", nm);
  if (kind < U_EXP || kind > U_SCALE) return fail(YR_E_INVALID, "%s: unknown kind %d", nm, kind);
  hipStream_t st = (hipStream_t)stream;
  return by_dtype(dtype, [&](auto dt) {
    hipLaunchKernelGGL((unary_kernel<decltype(dt)::value>), dim3(grid_for(n)), dim3(256), 0, st, (const uint16_t*)x,
                       (uint16_t*)y, (long long)n, kind, lo, hi);
    YR_CHECK_LAUNCH(nm);
    return YR_OK;
  });
}

int yr_hip_graph_binary(const void* a, const void* b, void* out, int ndim, const int64_t* dims_a,
                        const int64_t* dims_b, int kind, int dtype, void* stream) {
  const char* nm = "yr_hip_graph_binary";
  if (!a || !b || !out || !dims_a || !dims_b) return fail(YR_E_INVALID, "%s: null pointer", nm);
  if (ndim <= 0 || ndim > kMaxDims) return fail(YR_E_INVALID, "%s: %d dims (1..%d)", nm, ndim, kMaxDims);
  if (kind < B_ADD || kind > B_POW) return fail(YR_E_INVALID, "%s: unknown kind %d", nm, kind);
  BinaryArgs p;
  p.a = (const uint16_t*)a;
  p.b = (const uint16_t*)b;
  p.out = (uint16_t*)out;
  p.nd = ndim;
  p.kind = kind;
  long long sa = 1, sb = 1, n = 1;
  for (int d = ndim - 1; d >= 0; d--) {
    const long long da = dims_a[d], db = dims_b[d];
    if (da <= 0 || db <= 0 || (da != db && da != 1 && db != 1))
      return fail(YR_E_INVALID, "%s: dims %lld and %lld of axis %d do not broadcast", nm, da, db, d);
    p.dims[d] = da > db ? da : db;
    p.div[d] = fast_div((uint32_t)(p.dims[d] < (1ll << 31) ? p.dims[d] : 1));
    p.sa[d] = da == 1 && p.dims[d] > 1 ? 0 : sa;
    p.sb[d] = db == 1 && p.dims[d] > 1 ? 0 : sb;
    sa *= da;
    sb *= db;
    n *= p.dims[d];
  }
  p.n = n;
  hipStream_t st = (hipStream_t)stream;
  return by_dtype(dtype, [&](auto dt) {
    hipLaunchKernelGGL((binary_kernel<decltype(dt)::value>), dim3(grid_for(n)), dim3(256), 0, st, p);
    YR_CHECK_LAUNCH(nm);
    return YR_OK;
  });
}

int yr_hip_graph_ewise(const void* const* ins, int nin, void* out, int ndim, const int64_t* out_dims,
                       const int64_t* in_dims, int nprog, const int32_t* prog, const float* imm, int dtype,
                       void* stream) {
  const char* nm = "yr_hip_graph_ewise";
  if (!ins || !out || !out_dims || !in_dims || !prog || !imm) return fail(YR_E_INVALID, "%s: null pointer", nm);
  if (ndim <= 0 || ndim > kMaxDims) return fail(YR_E_INVALID, "%s: %d dims (1..%d)", nm, ndim, kMaxDims);
  if (nin <= 0 || nin > kEwIn) return fail(YR_E_INVALID, "%s: %d inputs (1..%d)", nm, nin, kEwIn);
  if (nprog <= 0 || nprog > kEwProg) return fail(YR_E_INVALID, "%s: %d instructions (1..%d)", nm, nprog, kEwProg);
  EwiseArgs p;
  memset(&p, 0, sizeof(p));
  long long n = 1;
  for (int d = 0; d < ndim; d++) {
    if (out_dims[d] <= 0) return fail(YR_E_INVALID, "%s: output dim %d", nm, d);
    p.div[d] = fast_div((uint32_t)out_dims[d]);
    n *= out_dims[d];
  }
  if (n >= (1ll << 31)) return fail(YR_E_INVALID, "%s: %lld elements (< 2^31)", nm, n);
  for (int k = 0; k < nin; k++) {
    if (!ins[k]) return fail(YR_E_INVALID, "%s: input %d is null", nm, k);
    p.in[k] = (const uint16_t*)ins[k];
    long long st = 1;
    for (int d = ndim - 1; d >= 0; d--) {
      const long long dk = in_dims[k * ndim + d];
      if (dk != 1 && dk != out_dims[d])
        return fail(YR_E_INVALID, "%s: input %d dim %d (%lld) does not broadcast to %lld", nm, k, d, dk,
                    (long long)out_dims[d]);
      p.s[k][d] = dk == 1 ? 0u : (uint32_t)st;
      st *= dk;
    }
  }
  for (int k = nin; k < kEwIn; k++) p.in[k] = p.in[0];
  bool defined[kEwRegs] = {};
  int nreg = 0;
  for (int j = 0; j < nprog; j++) {
    const int32_t* w = prog + 5 * j;  // {op, dst, a, b, kind}
    const int op = w[0], dst = w[1], a = w[2], b = w[3], kind = w[4];
    if (dst < 0 || dst >= kEwRegs) return fail(YR_E_INVALID, "%s: instruction %d: register %d", nm, j, dst);
    if (op == EW_LOAD) {
      if (a < 0 || a >= nin) return fail(YR_E_INVALID, "%s: instruction %d loads input %d", nm, j, a);
    } else if (op == EW_UNARY) {
      if (a < 0 || a >= kEwRegs || !defined[a] || kind < U_EXP || kind > U_SCALE)
        return fail(YR_E_INVALID, "%s: instruction %d: bad unary", nm, j);
    } else if (op == EW_BINARY) {
      if (a < 0 || a >= kEwRegs || b < 0 || b >= kEwRegs || !defined[a] || !defined[b] || kind < B_ADD ||
          kind > B_POW)
        return fail(YR_E_INVALID, "%s: instruction %d: bad binary", nm, j);
    } else {
      return fail(YR_E_INVALID, "%s: instruction %d: op %d", nm, j, op);
    }
    defined[dst] = true;
    if (dst + 1 > nreg) nreg = dst + 1;
    p.op[j] = op;
    p.dst[j] = dst;
    p.a[j] = a;
    p.b[j] = b;
    p.kind[j] = kind;
    p.lo[j] = imm[2 * j];
    p.hi[j] = imm[2 * j + 1];
  }
  p.out = (uint16_t*)out;
  p.n = (uint32_t)n;
  p.nd = ndim;
  p.nin = nin;
  p.nprog = nprog;
  hipStream_t st = (hipStream_t)stream;
  // the register file is selected by compares: the smallest that holds the program
  return by_dtype(dtype, [&](auto dt) {
    constexpr int D = decltype(dt)::value;
    // four elements per thread once the chip is full (amortizes the program
    // decode), one below that (latency-bound sizes want the waves)
    const bool big = n >= (1ll << 18);
    const int grid = grid_for(big ? (n + 3) / 4 : n);
#define YR_EW(NR_)                                                                               \
  if (big) hipLaunchKernelGGL((ewise_kernel<D, NR_, 4>), dim3(grid), dim3(256), 0, st, p);      \
  else hipLaunchKernelGGL((ewise_kernel<D, NR_, 1>), dim3(grid), dim3(256), 0, st, p);
    if (nreg <= 4) {
      YR_EW(4)
    } else if (nreg <= 8) {
      YR_EW(8)
    } else {
      YR_EW(kEwRegs)
    }
#undef YR_EW
    YR_CHECK_LAUNCH(nm);
    return YR_OK;
  });
}

int yr_hip_graph_reduction(const void* x, void* y, int64_t outer, int red, int64_t inner, int dtype, void* stream) {
  const char* nm = "yr_hip_graph_reduction";
  if (!x || !y || outer <= 0 || red <= 0 || inner <= 0) return fail(YR_E_INVALID, "%s: bad arguments", nm);
  return reduce_launch<false>(nm, x, y, outer, red, inner, dtype, (hipStream_t)stream);
}

int yr_hip_graph_reduction_max(const void* x, void* y, int64_t outer, int red, int64_t inner, int dtype,
                               void* stream) {
  const char* nm = "yr_hip_graph_reduction_max";
  if (!x || !y || outer <= 0 || red <= 0 || inner <= 0) return fail(YR_E_INVALID, "%s: bad arguments", nm);
  return reduce_launch<true>(nm, x, y, outer, red, inner, dtype, (hipStream_t)stream);
}

int yr_hip_graph_rmsnorm(const void* x, void* y, int rows, int n, float eps, int dtype, void* stream) {
  const char* nm = "yr_hip_graph_rmsnorm";
  if (!x || !y || rows <= 0 || n <= 0) return fail(YR_E_INVALID, "%s: bad arguments", nm);
  hipStream_t st = (hipStream_t)stream;
  return by_dtype(dtype, [&](auto dt) {
    hipLaunchKernelGGL((rmsnorm_kernel<decltype(dt)::value>), dim3(rows), dim3(256), 0, st, (const uint16_t*)x,
                       (uint16_t*)y, n, eps);
    YR_CHECK_LAUNCH(nm);
    return YR_OK;
  });
}

int yr_hip_graph_matmul(const void* a, const void* b, void* c, int batch, int m, int n, int k, int dtype,
                        void* stream) {
  const char* nm = "yr_hip_graph_matmul";
  if (!a || !b || !c) return fail(YR_E_INVALID, "%s: null pointer", nm);
  if (batch <= 0 || m <= 0 || n <= 0 || k <= 0) return fail(YR_E_INVALID, "%s: bad shape", nm);
  if (n % 8 || k % 8) return fail(YR_E_INVALID, "%s: N and K must be multiples of 8 (got %d, %d)", nm, n, k);
  if (batch > 65535 || (m + MM_T - 1) / MM_T > 65535) return fail(YR_E_INVALID, "%s: grid too large", nm);
  hipStream_t st = (hipStream_t)stream;
  dim3 grid((n + MM_T - 1) / MM_T, (m + MM_T - 1) / MM_T, batch);
  return by_dtype(dtype, [&](auto dt) {
    hipLaunchKernelGGL((matmul_kernel<decltype(dt)::value>), grid, dim3(256), 0, st, (const uint16_t*)a,
                       (const uint16_t*)b, (uint16_t*)c, m, n, k, (long long)m * k, (long long)k * n,
                       (long long)m * n);
    YR_CHECK_LAUNCH(nm);
    return YR_OK;
  });
}

}  // extern "C"
