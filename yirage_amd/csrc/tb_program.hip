// One launch per customized operator: a threadblock graph (the reference's
// TB graph of a customized op, src/threadblock/graph.cc; the role its
// transpiler gives to generated CUDA, src/transpiler/transpile.cc:370-720)
// run by a small tile program interpreter.  A workgroup is one block of the
// customized op's grid; every tile lives in LDS for the whole launch (no
// block tensor reaches HBM), inputs are cut from the device tensors by
// input_map / forloop_dim each iteration, outputs are placed by output_map /
// forloop_dim.  Tiles are stored in the 16-bit type, so each operator's
// result is rounded once (as the transpiled element ops do); math is fp32,
// and accumulators keep fp32 buffers over the iterations, rounded once when
// they are finalised.  Tiles whose lifetimes do not overlap share LDS.
//
// Program words (int32), see yr_hip_tb_program in include/yirage_hip.h:
//   header  {version, dtype, R, n_tensors, n_inputs, n_ops, n_outputs,
//            lds_bytes, reduction_dimx, gx, gy, gz}
//   tensors n_tensors x {lds_byte_offset, ndim, d0, d1, d2, d3, wide}
//            (wide: an fp32 accumulator buffer; every other tile is 16-bit)
//   inputs  n_inputs x {tensor, input_index, gdims[4], im[3], forloop_dim}
//           (device tensors dense row-major, rank = the tile's)
//   ops     n_ops x {kind, out, in0, in1, a0, a1, a2, phase, acc}
//   outputs n_outputs x {tensor, output_index, gdims[4], om[3], forloop_dim,
//            post (1: the tile is final only after the loop)}
#include <math.h>
#include <string.h>

#include "yr_common.h"

namespace yr {
namespace tbp {

constexpr int kVersion = 1;
constexpr int kHdr = 12, kTw = 7, kIw = 10, kOw = 11, kRw = 9;
constexpr int kMaxWords = 800, kMaxIn = 8, kMaxOut = 4, kMaxDim = 4;
constexpr int kThreads = 1024;
constexpr int kMaxLdsBytes = 160 * 1024 - 256;  // the tiles' share (block reductions keep a few words)

enum OpKind { K_UNARY = 1, K_BINARY = 2, K_MATMUL = 3, K_REDUCE = 4, K_REDMAX = 5, K_RMSNORM = 6, K_CONCAT = 7,
              K_ACC = 8 };
enum UnaryKind { U_EXP = 0, U_SILU = 1, U_GELU = 2, U_RELU = 3, U_CLAMP = 4, U_SQRT = 5, U_SQUARE = 6, U_SCALE = 7 };
enum BinaryKind { B_ADD = 0, B_MUL = 1, B_DIV = 2, B_POW = 3, B_SUB = 4 };
enum AccKind { A_NONE = 0, A_SUM = 1, A_TODIMX = 2, A_RMS = 3, A_MEAN = 4, A_MAX = 5, A_RESCALE = 6,
               A_RESCALE_SUM = 7 };

struct Args {
  const uint16_t* in[kMaxIn];
  uint16_t* out[kMaxOut];
  int32_t w[kMaxWords];
};

struct Tile {
  int off, nd, d[kMaxDim], n, wide;  // off in bytes; wide: fp32 (accumulator buffers), else 16-bit
};

__device__ __forceinline__ Tile tile_of(const int32_t* w, int t) {
  const int32_t* p = w + kHdr + t * kTw;
  Tile x;
  x.off = p[0];
  x.nd = p[1];
  x.wide = p[6];
  x.n = 1;
#pragma unroll
  for (int i = 0; i < kMaxDim; i++) {
    x.d[i] = i < x.nd ? p[2 + i] : 1;
    x.n *= x.d[i];
  }
  return x;
}

// a[i] for a runtime i without indexing the array (a runtime index would put
// the array, and the tile holding it, in per-lane scratch memory)
__device__ __forceinline__ int dsel(const int (&a)[kMaxDim], int i) {
  return i == 0 ? a[0] : i == 1 ? a[1] : i == 2 ? a[2] : a[3];
}
__device__ __forceinline__ void dadd(int (&a)[kMaxDim], int i, int v) {
#pragma unroll
  for (int q = 0; q < kMaxDim; q++)
    if (q == i) a[q] += v;
}

// element i of a tile as fp32 / stored (a 16-bit tile rounds: one rounding
// per operator)
template <int DT>
__device__ __forceinline__ float tld(const char* lds, const Tile& t, int i) {
  return t.wide ? reinterpret_cast<const float*>(lds + t.off)[i]
                : ld_elem<DT>(reinterpret_cast<const uint16_t*>(lds + t.off)[i]);
}
template <int DT>
__device__ __forceinline__ void tst(char* lds, const Tile& t, int i, float v) {
  if (t.wide) reinterpret_cast<float*>(lds + t.off)[i] = v;
  else reinterpret_cast<uint16_t*>(lds + t.off)[i] = (uint16_t)st_elem<DT>(v);
}

// coordinates of element e of a row-major tile
__device__ __forceinline__ void coords(const Tile& t, int e, int (&c)[kMaxDim]) {
#pragma unroll
  for (int i = kMaxDim - 1; i >= 0; i--) {
    if (i < t.nd) {
      c[i] = e % t.d[i];
      e /= t.d[i];
    } else {
      c[i] = 0;
    }
  }
}

// element of tile t at coordinates c (dims of size 1 broadcast)
__device__ __forceinline__ int index_bcast(const Tile& t, const int (&c)[kMaxDim]) {
  int idx = 0;
#pragma unroll
  for (int i = 0; i < kMaxDim; i++)
    if (i < t.nd) idx = idx * t.d[i] + (t.d[i] == 1 ? 0 : c[i]);
  return idx;
}

__device__ __forceinline__ float unary(int kind, float a, float lo, float hi) {
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
__device__ __forceinline__ float binary(int kind, float x, float y) {
  switch (kind) {
    case B_ADD: return x + y;
    case B_MUL: return x * y;
    case B_DIV: return x / y;
    case B_SUB: return x - y;
    default: return powf(x, y);
  }
}

// start of this block's (iteration's) tile along each dim of a device tensor
__device__ __forceinline__ void tile_start(const int32_t* r, const Tile& t, int it, int (&s)[kMaxDim]) {
  const int gd[kMaxDim] = {r[2], r[3], r[4], r[5]};
  const int b[3] = {(int)blockIdx.x, (int)blockIdx.y, (int)blockIdx.z};
  const int g[3] = {(int)gridDim.x, (int)gridDim.y, (int)gridDim.z};
#pragma unroll
  for (int i = 0; i < kMaxDim; i++) s[i] = 0;
#pragma unroll
  for (int a = 0; a < 3; a++) {
    const int m = r[6 + a];
    if (m >= 0) dadd(s, m, b[a] * (dsel(gd, m) / g[a]));
  }
  const int fd = r[9];
  if (fd >= 0) dadd(s, fd, it * dsel(t.d, fd));
}

// device element offset of tile element e
__device__ __forceinline__ long long dev_index(const int32_t* r, const Tile& t, const int (&s)[kMaxDim], int e) {
  int c[kMaxDim];
  coords(t, e, c);
  long long g = 0;
#pragma unroll
  for (int i = 0; i < kMaxDim; i++)
    if (i < t.nd) g = g * r[2 + i] + (s[i] + c[i]);
  return g;
}

// sum / max over the 64 lanes of a wave (every lane gets the result)
__device__ __forceinline__ float wave_red(float v, bool mx) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) {
    const float u = __shfl_xor(v, o);
    v = mx ? fmaxf(v, u) : v + u;
  }
  return v;
}

// one float per wave for block-wide reductions
__shared__ float tb_red[kThreads / 64];

// sum / max over the whole block (every thread gets the result; all threads
// must call it)
__device__ __forceinline__ float block_red(float v, bool mx) {
  v = wave_red(v, mx);
  if ((threadIdx.x & 63) == 0) tb_red[threadIdx.x >> 6] = v;
  __syncthreads();
  float r = tb_red[0];
#pragma unroll
  for (int i = 1; i < kThreads / 64; i++) r = mx ? fmaxf(r, tb_red[i]) : r + tb_red[i];
  __syncthreads();  // tb_red is reused by the next call
  return r;
}

// whole 16-byte pieces: the tile's and the device tensor's rows hold whole
// groups of 8 elements, the tile starts on one, and both base addresses are
// 16-byte aligned
__device__ __forceinline__ bool vec8(const Tile& t, const int32_t* r, const int (&s)[kMaxDim], const void* dev) {
  const int l = t.nd - 1;
  return ((dsel(t.d, l) | r[2 + l] | dsel(s, l)) & 7) == 0 && (t.off & 15) == 0 && (reinterpret_cast<uintptr_t>(dev) & 15) == 0;
}

template <int DT>
__device__ __forceinline__ f32x4 mfma16(uint4 a, uint4 b, f32x4 c) {
  if constexpr (DT == DT_BF16)
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8v, a), __builtin_bit_cast(bf16x8v, b), c,
                                                   0, 0, 0);
  else
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8v, a), __builtin_bit_cast(f16x8v, b), c, 0,
                                                  0, 0);
}

// 16 bytes per lane from global memory straight into LDS: lane l's data
// lands at lds_base + 16 l (lds_base wave-uniform)
__device__ __forceinline__ void lds_load16(const uint16_t* g, uint16_t* lds_base) {
  __builtin_amdgcn_global_load_lds(
      (const __attribute__((address_space(1))) void*)(g),
      reinterpret_cast<__attribute__((address_space(3))) void*>(
          reinterpret_cast<__attribute__((address_space(3))) char*>(reinterpret_cast<uintptr_t>(lds_base))),
      16, 0, 0);
}

template <int DT>
__device__ __forceinline__ void load_input(const Args& A, const int32_t* w, const int32_t* r, int it, char* lds) {
  const Tile t = tile_of(w, r[0]);
  const uint16_t* src = A.in[r[1]];
  uint16_t* dst = reinterpret_cast<uint16_t*>(lds + t.off);  // input tiles are 16-bit
  int s[kMaxDim];
  tile_start(r, t, it, s);
  if (vec8(t, r, s, src)) {  // 16-byte row pieces straight into LDS, 64 consecutive pieces per wave
    const int nc = t.n >> 3, lane = threadIdx.x & 63;
    for (int g0 = (threadIdx.x >> 6) * 64; g0 < nc; g0 += kThreads) {
      const int c = g0 + lane;
      if (c < nc) lds_load16(src + dev_index(r, t, s, c << 3), dst + (g0 << 3));
    }
    return;  // (the caller waits for the loads before its barrier)
  }
  for (int e = threadIdx.x; e < t.n; e += kThreads) dst[e] = src[dev_index(r, t, s, e)];
}

template <int DT>
__device__ __forceinline__ void store_output(const Args& A, const int32_t* w, const int32_t* r, int it, const char* lds) {
  const Tile t = tile_of(w, r[0]);
  uint16_t* dst = A.out[r[1]];
  int s[kMaxDim];
  tile_start(r, t, it, s);
  if (vec8(t, r, s, dst)) {
    for (int c = threadIdx.x; c < (t.n >> 3); c += kThreads) {
      uint4 v;
      if (t.wide) {  // 8 fp32 values, each rounded once
        const float* f = reinterpret_cast<const float*>(lds + t.off) + (c << 3);
        v.x = st_elem<DT>(f[0]) | (st_elem<DT>(f[1]) << 16);
        v.y = st_elem<DT>(f[2]) | (st_elem<DT>(f[3]) << 16);
        v.z = st_elem<DT>(f[4]) | (st_elem<DT>(f[5]) << 16);
        v.w = st_elem<DT>(f[6]) | (st_elem<DT>(f[7]) << 16);
      } else {  // already 16-bit values of the type
        v = *reinterpret_cast<const uint4*>(lds + t.off + (c << 4));
      }
      *reinterpret_cast<uint4*>(dst + dev_index(r, t, s, c << 3)) = v;
    }
    return;
  }
  for (int e = threadIdx.x; e < t.n; e += kThreads) dst[dev_index(r, t, s, e)] = (uint16_t)st_elem<DT>(tld<DT>(lds, t, e));
}

__device__ __forceinline__ float fbits(int32_t b) { return __int_as_float(b); }

// one operator over its output tile, all threads; fp32 math
template <int DT>
__device__ __forceinline__ void exec_op(const int32_t* w, const int32_t* o, char* lds) {
  const int kind = o[0];
  const Tile to = tile_of(w, o[1]);
  const Tile ta = tile_of(w, o[2]);
  switch (kind) {
    case K_UNARY: {
      const float lo = fbits(o[5]), hi = fbits(o[6]);
      for (int e = threadIdx.x; e < to.n; e += kThreads) tst<DT>(lds, to, e, unary(o[4], tld<DT>(lds, ta, e), lo, hi));
      break;
    }
    case K_BINARY: {
      const Tile tb = tile_of(w, o[3]);
      if (ta.n == to.n && tb.n == to.n) {  // no broadcast: the operands have the output's shape
        for (int e = threadIdx.x; e < to.n; e += kThreads)
          tst<DT>(lds, to, e, binary(o[4], tld<DT>(lds, ta, e), tld<DT>(lds, tb, e)));
        break;
      }
      for (int e = threadIdx.x; e < to.n; e += kThreads) {
        int c[kMaxDim];
        coords(to, e, c);
        tst<DT>(lds, to, e, binary(o[4], tld<DT>(lds, ta, index_bcast(ta, c)), tld<DT>(lds, tb, index_bcast(tb, c))));
      }
      break;
    }
    case K_MATMUL: {  // a [.., M, K] x b [.., K, N]
      const Tile tb = tile_of(w, o[3]);
      const int M = dsel(ta.d, ta.nd - 2), K = dsel(ta.d, ta.nd - 1), N = dsel(tb.d, tb.nd - 1);
      if (!ta.wide && !tb.wide && ((M | N) & 15) == 0 && (K & 31) == 0 && (ta.off & 15) == 0) {
        // 16 x 16 output tiles on MFMA (16x16x32), one wave per tile.  Lane l:
        // A = row l % 16, k 8 (l / 16) .. + 7 (one 16-byte LDS read); B =
        // column l % 16, the same 8 k; result rows 4 (l / 16) + i, column l % 16
        const int lane = threadIdx.x & 63, r16 = lane & 15, kg = (lane >> 4) * 8;
        const int mt = M >> 4, nt = N >> 4, per = mt * nt, tiles = (to.n / (M * N)) * per;
        const uint16_t* A_ = reinterpret_cast<const uint16_t*>(lds + ta.off);
        const uint16_t* B_ = reinterpret_cast<const uint16_t*>(lds + tb.off);
        for (int t = threadIdx.x >> 6; t < tiles; t += kThreads / 64) {
          const int bt = t / per, m0 = (t % per) / nt * 16, n0 = (t % nt) * 16;
          const uint16_t* ap = A_ + (bt * M + m0 + r16) * K + kg;
          const uint16_t* bp = B_ + bt * K * N + kg * N + n0 + r16;
          f32x4 c = {0.f, 0.f, 0.f, 0.f};
          for (int k0 = 0; k0 < K; k0 += 32) {
            const uint4 a = *reinterpret_cast<const uint4*>(ap + k0);
            const uint16_t* q = bp + k0 * N;
            const uint4 b = {q[0] | ((uint32_t)q[N] << 16), q[2 * N] | ((uint32_t)q[3 * N] << 16),
                             q[4 * N] | ((uint32_t)q[5 * N] << 16), q[6 * N] | ((uint32_t)q[7 * N] << 16)};
            c = mfma16<DT>(a, b, c);
          }
#pragma unroll
          for (int i = 0; i < 4; i++) tst<DT>(lds, to, (bt * M + m0 + (lane >> 4) * 4 + i) * N + n0 + r16, c[i]);
        }
        break;
      }
      for (int e = threadIdx.x; e < to.n; e += kThreads) {
        const int n = e % N, m = (e / N) % M, bt = e / (M * N);
        const int ar = (bt * M + m) * K, bc = bt * K * N + n;
        float s = 0.f;
        for (int k = 0; k < K; k++) s = fmaf(tld<DT>(lds, ta, ar + k), tld<DT>(lds, tb, bc + k * N), s);
        tst<DT>(lds, to, e, s);
      }
      break;
    }
    case K_REDUCE:    // sum over dim a0 down to a1 elements (element j adds j, j + a1, ...)
    case K_REDMAX: {  // max over dim a0
      const int dim = o[4], to_n = kind == K_REDUCE ? o[5] : 1;
      const int L = dsel(ta.d, dim);
      int inner = 1;
#pragma unroll
      for (int i = 0; i < kMaxDim; i++)
        if (i > dim && i < ta.nd) inner *= ta.d[i];
      const bool mx = kind == K_REDMAX;
      if (L / to_n >= kThreads && to.n < kThreads / 64) {  // few long reductions: the whole block on each
        for (int e = 0; e < to.n; e++) {
          const int in_ = e % inner, j = (e / inner) % to_n, ou = e / (inner * to_n);
          const int base = ou * L * inner + in_;
          float s = mx ? -INFINITY : 0.f;
          for (int r = j + threadIdx.x * to_n; r < L; r += kThreads * to_n) {
            const float v = tld<DT>(lds, ta, base + r * inner);
            s = mx ? fmaxf(s, v) : s + v;
          }
          s = block_red(s, mx);
          if (threadIdx.x == 0) tst<DT>(lds, to, e, s);
        }
        break;
      }
      if (L / to_n >= 64) {  // long reductions: one wave per output
        const int lane = threadIdx.x & 63;
        for (int e = threadIdx.x >> 6; e < to.n; e += kThreads / 64) {
          const int in_ = e % inner, j = (e / inner) % to_n, ou = e / (inner * to_n);
          const int base = ou * L * inner + in_;
          float s = mx ? -INFINITY : 0.f;
          for (int r = j + lane * to_n; r < L; r += 64 * to_n) {
            const float v = tld<DT>(lds, ta, base + r * inner);
            s = mx ? fmaxf(s, v) : s + v;
          }
          s = wave_red(s, mx);
          if (lane == 0) tst<DT>(lds, to, e, s);
        }
        break;
      }
      for (int e = threadIdx.x; e < to.n; e += kThreads) {
        const int in_ = e % inner, j = (e / inner) % to_n, ou = e / (inner * to_n);
        const int base = ou * L * inner + in_;
        float s = mx ? -INFINITY : 0.f;
        for (int r = j; r < L; r += to_n) {
          const float v = tld<DT>(lds, ta, base + r * inner);
          s = mx ? fmaxf(s, v) : s + v;
        }
        tst<DT>(lds, to, e, s);
      }
      break;
    }
    case K_RMSNORM: {  // rows of the last dim: x * rsqrt(mean(x^2) + eps), one wave per row
      const int n = dsel(ta.d, ta.nd - 1), rows = to.n / n, lane = threadIdx.x & 63;
      const float eps = fbits(o[5]);
      if (rows < kThreads / 64 && n >= kThreads) {  // few long rows: the whole block on each
        for (int row = 0; row < rows; row++) {
          const int b = row * n;
          float ss = 0.f;
          for (int i = threadIdx.x; i < n; i += kThreads) {
            const float v = tld<DT>(lds, ta, b + i);
            ss += v * v;
          }
          const float sc = rsqrtf(block_red(ss, false) / (float)n + eps);
          for (int i = threadIdx.x; i < n; i += kThreads) tst<DT>(lds, to, b + i, tld<DT>(lds, ta, b + i) * sc);
        }
        break;
      }
      for (int row = threadIdx.x >> 6; row < rows; row += kThreads / 64) {
        const int b = row * n;
        float ss = 0.f;
        for (int i = lane; i < n; i += 64) {
          const float v = tld<DT>(lds, ta, b + i);
          ss += v * v;
        }
        const float sc = rsqrtf(wave_red(ss, false) / (float)n + eps);
        for (int i = lane; i < n; i += 64) tst<DT>(lds, to, b + i, tld<DT>(lds, ta, b + i) * sc);
      }
      break;
    }
    case K_CONCAT: {  // a then b along dim a0
      const Tile tb = tile_of(w, o[3]);
      const int dim = o[4];
      for (int e = threadIdx.x; e < to.n; e += kThreads) {
        int c[kMaxDim];
        coords(to, e, c);
        const int ad = dsel(ta.d, dim);
        const bool first = dsel(c, dim) < ad;
        if (!first) dadd(c, dim, -ad);
        const Tile ts = first ? ta : tb;
        int idx = 0;
#pragma unroll
        for (int i = 0; i < kMaxDim; i++)
          if (i < ts.nd) idx = idx * ts.d[i] + c[i];
        tst<DT>(lds, to, e, tld<DT>(lds, ts, idx));
      }
      break;
    }
    default:
      break;
  }
}

// accumulator update (per iteration): the fp32 buffer, the input tile's shape
template <int DT>
__device__ __forceinline__ void acc_update(const int32_t* w, const int32_t* o, char* lds) {
  const Tile tx = tile_of(w, o[2]), ta = tile_of(w, o[8]);
  float* acc = reinterpret_cast<float*>(lds + ta.off);
  const int kind = o[4];
  if (kind == A_RESCALE || kind == A_RESCALE_SUM) {
    const Tile tr = tile_of(w, o[3]);
    for (int e = threadIdx.x; e < tx.n; e += kThreads) {
      int c[kMaxDim];
      coords(tx, e, c);
      acc[e] = acc[e] * tld<DT>(lds, tr, index_bcast(tr, c)) + tld<DT>(lds, tx, e);
    }
    return;
  }
  for (int e = threadIdx.x; e < tx.n; e += kThreads) {
    const float v = tld<DT>(lds, tx, e);
    if (kind == A_MAX) acc[e] = fmaxf(acc[e], v);
    else acc[e] += kind == A_RMS ? v * v : v;
  }
}

__device__ __forceinline__ void acc_init(const int32_t* w, const int32_t* o, char* lds) {
  const Tile ta = tile_of(w, o[8]);
  float* acc = reinterpret_cast<float*>(lds + ta.off);
  const float v = o[4] == A_MAX ? -INFINITY : 0.f;
  for (int e = threadIdx.x; e < ta.n; e += kThreads) acc[e] = v;
}

// after the loop: the accumulator's value into its (16-bit) output tile
template <int DT>
__device__ __forceinline__ void acc_final(const int32_t* w, const int32_t* o, char* lds, int R, int dimx) {
  const Tile tx = tile_of(w, o[2]), ta = tile_of(w, o[8]), to = tile_of(w, o[1]);
  const float* acc = reinterpret_cast<const float*>(lds + ta.off);
  const int kind = o[4];
  const int n = dsel(tx.d, tx.nd - 1);
  const bool red = !(kind == A_NONE || kind == A_MAX || kind == A_RESCALE);
  const int to_n = kind == A_TODIMX ? dimx : 1;
  if (red && n / to_n >= kThreads && to.n < kThreads / 64) {  // few long row sums: the whole block on each
    for (int e = 0; e < to.n; e++) {
      const float* p = acc + (size_t)(e / to_n) * n;
      float s = 0.f;
      for (int i = e % to_n + threadIdx.x * to_n; i < n; i += kThreads * to_n) s += p[i];
      s = block_red(s, false);
      if (kind == A_MEAN) s /= (float)(n * R);
      else if (kind == A_RMS) s = sqrtf(s / (float)(n * R));
      if (threadIdx.x == 0) tst<DT>(lds, to, e, s);
    }
    return;
  }
  if (red && n / to_n >= 64) {  // long row sums: one wave per output
    const int lane = threadIdx.x & 63;
    for (int e = threadIdx.x >> 6; e < to.n; e += kThreads / 64) {
      const float* p = acc + (size_t)(e / to_n) * n;
      float s = 0.f;
      for (int i = e % to_n + lane * to_n; i < n; i += 64 * to_n) s += p[i];
      s = wave_red(s, false);
      if (kind == A_MEAN) s /= (float)(n * R);
      else if (kind == A_RMS) s = sqrtf(s / (float)(n * R));
      if (lane == 0) tst<DT>(lds, to, e, s);
    }
    return;
  }
  for (int e = threadIdx.x; e < to.n; e += kThreads) {
    float v;
    if (kind == A_NONE || kind == A_MAX || kind == A_RESCALE) {
      v = acc[e];
    } else {
      const int j = e % to_n, row = e / to_n;
      const float* p = acc + (size_t)row * n;
      float s = 0.f;
      for (int i = j; i < n; i += to_n) s += p[i];
      if (kind == A_MEAN) s /= (float)(n * R);
      else if (kind == A_RMS) s = sqrtf(s / (float)(n * R));
      v = s;
    }
    tst<DT>(lds, to, e, v);
  }
}

template <int DT>
__global__ __launch_bounds__(kThreads) void tb_program_kernel(Args A) {
  extern __shared__ __attribute__((aligned(16))) char lds[];
  const int32_t* w = A.w;
  const int R = w[2], nt = w[3], ni = w[4], no = w[5], nout = w[6], dimx = w[8];
  const int32_t* ins = w + kHdr + nt * kTw;
  const int32_t* ops = ins + ni * kIw;
  const int32_t* outs = ops + no * kRw;
  for (int it = 0; it < R; it++) {
    for (int i = 0; i < ni; i++)
      if (it == 0 || ins[i * kIw + 9] >= 0) load_input<DT>(A, w, ins + i * kIw, it, lds);
    __builtin_amdgcn_s_waitcnt(0x0f70);  // vmcnt(0): this wave's loads into LDS have landed
    if (it == 0) {  // (accumulator buffers may reuse tiles that are dead by now: after the loads)
      __syncthreads();
      for (int i = 0; i < no; i++)
        if (ops[i * kRw] == K_ACC) acc_init(w, ops + i * kRw, lds);
    }
    __syncthreads();
    for (int i = 0; i < no; i++) {
      const int32_t* o = ops + i * kRw;
      if (o[7] != 0) continue;  // after the loop
      if (o[0] == K_ACC) acc_update<DT>(w, o, lds);
      else exec_op<DT>(w, o, lds);
      __syncthreads();
    }
    // outputs placed per iteration
    for (int i = 0; i < nout; i++) {
      const int32_t* r = outs + i * kOw;
      if (r[9] >= 0 && r[10] == 0) store_output<DT>(A, w, r, it, lds);
    }
    __syncthreads();  // the tiles are read before the next iteration's loads replace them
  }
  for (int i = 0; i < no; i++)
    if (ops[i * kRw] == K_ACC) acc_final<DT>(w, ops + i * kRw, lds, R, dimx);
  __syncthreads();
  for (int i = 0; i < no; i++) {
    const int32_t* o = ops + i * kRw;
    if (o[7] == 0) continue;
    exec_op<DT>(w, o, lds);
    __syncthreads();
  }
  for (int i = 0; i < nout; i++) {
    const int32_t* r = outs + i * kOw;
    if (r[9] >= 0 && r[10] == 0) continue;  // stored in the loop
    // a final tile placed along the forloop dim goes to every iteration's slot
    const int reps = r[9] >= 0 ? R : 1;
    for (int it = 0; it < reps; it++) store_output<DT>(A, w, r, it, lds);
  }
}

// Host-side check of a program against the launch: every tile inside the
// LDS budget, every tensor reference, every op's shapes and every device
// tile access in bounds, so the kernel never indexes outside what it was
// given.
static int check_program(const int32_t* w, int nw, int n_in, int n_out, int gx, int gy, int gz, const char* nm) {
  auto bad = [&](const char* what) { return fail(YR_E_INVALID, "%s: bad program (%s)", nm, what); };
  if (nw < kHdr || nw > kMaxWords) return bad("size");
  const int R = w[2], nt = w[3], ni = w[4], no = w[5], nout = w[6], lf = w[7], dimx = w[8];
  if (w[0] != kVersion) return bad("version");
  if (R < 1 || nt < 1 || ni < 1 || ni > kMaxIn || no < 0 || nout < 1 || nout > kMaxOut) return bad("counts");
  if (kHdr + nt * kTw + ni * kIw + no * kRw + nout * kOw != nw) return bad("length");
  if (lf < 1 || lf > kMaxLdsBytes || dimx < 1) return bad("lds / dimx");
  if (ni != n_in || nout != n_out) return bad("input / output count");
  if (w[9] != gx || w[10] != gy || w[11] != gz) return bad("grid");
  Tile T[kMaxWords / kTw];
  for (int t = 0; t < nt; t++) {
    const int32_t* p = w + kHdr + t * kTw;
    Tile& x = T[t];
    x.off = p[0];
    x.nd = p[1];
    x.wide = p[6];
    if (x.nd < 1 || x.nd > kMaxDim || (x.wide != 0 && x.wide != 1)) return bad("tile rank");
    long long n = 1;
    for (int i = 0; i < kMaxDim; i++) {
      x.d[i] = i < x.nd ? p[2 + i] : 1;
      if (x.d[i] < 1) return bad("tile dim");
      n *= x.d[i];
    }
    const int es = x.wide ? 4 : 2;
    if (x.off < 0 || x.off % es || x.off + n * es > lf) return bad("tile outside the LDS budget");
    x.n = (int)n;
  }
  const int g[3] = {gx, gy, gz};
  auto check_io = [&](const int32_t* r, int count, bool is_in) -> bool {
    if (r[0] < 0 || r[0] >= nt || r[1] < 0 || r[1] >= count) return false;
    const Tile& x = T[r[0]];
    if (x.wide) return false;
    const int fd = r[9];
    if (fd >= x.nd || fd < -1) return false;
    for (int d = 0; d < x.nd; d++) {
      const int gd = r[2 + d];
      if (gd < 1) return false;
      long long block = gd;
      int cuts = 0;
      for (int a = 0; a < 3; a++) {
        const int m = r[6 + a];
        if (m < -1 || m >= x.nd) return false;
        if (m == d) {
          if (gd % g[a]) return false;
          block = gd / g[a];
          cuts++;
        }
      }
      if (cuts > 1) return false;
      const long long span = (long long)x.d[d] * (d == fd ? R : 1);
      if (span > block) return false;
    }
    (void)is_in;
    return true;
  };
  const int32_t* ins = w + kHdr + nt * kTw;
  for (int i = 0; i < ni; i++)
    if (!check_io(ins + i * kIw, n_in, true)) return bad("input tile outside its tensor");
  const int32_t* ops = ins + ni * kIw;
  auto same = [&](const Tile& a, const Tile& b) {
    if (a.nd != b.nd) return false;
    for (int i = 0; i < a.nd; i++)
      if (a.d[i] != b.d[i]) return false;
    return true;
  };
  for (int i = 0; i < no; i++) {
    const int32_t* o = ops + i * kRw;
    const int k = o[0];
    auto tid_ok = [&](int t) { return t >= 0 && t < nt; };
    if (!tid_ok(o[1]) || !tid_ok(o[2]) || (o[7] != 0 && o[7] != 1)) return bad("op tensor");
    const Tile &to = T[o[1]], &ta = T[o[2]];
    if (to.wide || ta.wide || (k != K_UNARY && k != K_RMSNORM && k != K_REDUCE && k != K_REDMAX && o[3] >= 0 &&
                               tid_ok(o[3]) && T[o[3]].wide))
      return bad("16-bit operator tiles");
    switch (k) {
      case K_UNARY:
        if (!same(to, ta) || o[4] < 0 || o[4] > U_SCALE) return bad("unary");
        break;
      case K_BINARY: {
        if (!tid_ok(o[3]) || o[4] < 0 || o[4] > B_SUB) return bad("binary");
        const Tile& tb = T[o[3]];
        if (ta.nd != to.nd || tb.nd != to.nd) return bad("binary rank");
        for (int d = 0; d < to.nd; d++)
          if ((ta.d[d] != to.d[d] && ta.d[d] != 1) || (tb.d[d] != to.d[d] && tb.d[d] != 1) ||
              to.d[d] != (ta.d[d] > tb.d[d] ? ta.d[d] : tb.d[d]))
            return bad("binary dims");
        break;
      }
      case K_MATMUL: {
        if (!tid_ok(o[3])) return bad("matmul");
        const Tile& tb = T[o[3]];
        if (ta.nd < 2 || tb.nd != ta.nd || to.nd != ta.nd) return bad("matmul rank");
        for (int d = 0; d < ta.nd - 2; d++)
          if (ta.d[d] != tb.d[d] || to.d[d] != ta.d[d]) return bad("matmul batch");
        if (tb.d[ta.nd - 2] != ta.d[ta.nd - 1] || to.d[ta.nd - 2] != ta.d[ta.nd - 2] || to.d[ta.nd - 1] != tb.d[ta.nd - 1])
          return bad("matmul dims");
        break;
      }
      case K_REDUCE:
      case K_REDMAX: {
        const int dim = o[4], to_n = k == K_REDUCE ? o[5] : 1;
        if (dim < 0 || dim >= ta.nd || to.nd != ta.nd || to_n < 1 || ta.d[dim] % to_n) return bad("reduction");
        for (int d = 0; d < ta.nd; d++)
          if (to.d[d] != (d == dim ? to_n : ta.d[d])) return bad("reduction dims");
        break;
      }
      case K_RMSNORM:
        if (!same(to, ta)) return bad("rms_norm");
        break;
      case K_CONCAT: {
        if (!tid_ok(o[3])) return bad("concat");
        const Tile& tb = T[o[3]];
        const int dim = o[4];
        if (dim < 0 || dim >= to.nd || ta.nd != to.nd || tb.nd != to.nd) return bad("concat rank");
        for (int d = 0; d < to.nd; d++)
          if (to.d[d] != (d == dim ? ta.d[d] + tb.d[d] : ta.d[d]) || (d != dim && tb.d[d] != ta.d[d]))
            return bad("concat dims");
        break;
      }
      case K_ACC: {
        if (!tid_ok(o[8]) || o[7] != 0 || o[4] < A_NONE || o[4] > A_RESCALE_SUM) return bad("accumulator");
        const Tile& tc = T[o[8]];
        if (!same(tc, ta) || !tc.wide) return bad("accumulator buffer");
        const int n = ta.d[ta.nd - 1];
        for (int d = 0; d < ta.nd - 1; d++)
          if (to.nd != ta.nd || to.d[d] != ta.d[d]) return bad("accumulator output");
        const int kind = o[4];
        const int last = kind == A_NONE || kind == A_MAX || kind == A_RESCALE ? n : kind == A_TODIMX ? dimx : 1;
        if (to.d[ta.nd - 1] != last || (kind == A_TODIMX && n % dimx)) return bad("accumulator output dims");
        if (kind == A_RESCALE || kind == A_RESCALE_SUM) {
          if (!tid_ok(o[3])) return bad("rescale");
          const Tile& tr = T[o[3]];
          if (tr.nd != ta.nd || tr.d[ta.nd - 1] != 1) return bad("rescale dims");
          for (int d = 0; d < ta.nd - 1; d++)
            if (tr.d[d] != ta.d[d]) return bad("rescale dims");
        }
        break;
      }
      default:
        return bad("op kind");
    }
  }
  const int32_t* outs = ops + no * kRw;
  for (int i = 0; i < nout; i++)
    if (!check_io(outs + i * kOw, n_out, false) || (outs[i * kOw + 10] != 0 && outs[i * kOw + 10] != 1))
      return bad("output tile outside its tensor");
  return YR_OK;
}

}  // namespace tbp
}  // namespace yr

extern "C" int yr_hip_tb_program(const int32_t* program, int n_words, const void* const* ins, int n_in,
                                 void* const* outs, int n_out, int gx, int gy, int gz, int dtype, void* stream) {
  using namespace yr;
  using namespace yr::tbp;
  const char* nm = "yr_hip_tb_program";
  if (!program || !ins || !outs) return fail(YR_E_INVALID, "%s: null pointer", nm);
  if (dtype != YR_DTYPE_F16 && dtype != YR_DTYPE_BF16) return fail(YR_E_INVALID, "%s: dtype", nm);
  if (gx < 1 || gy < 1 || gz < 1 || gy > 65535 || gz > 65535) return fail(YR_E_INVALID, "%s: grid", nm);
  if (n_in < 1 || n_in > kMaxIn || n_out < 1 || n_out > kMaxOut) return fail(YR_E_INVALID, "%s: %d inputs, %d outputs", nm, n_in, n_out);
  for (int i = 0; i < n_in; i++)
    if (!ins[i]) return fail(YR_E_INVALID, "%s: null input %d", nm, i);
  for (int i = 0; i < n_out; i++)
    if (!outs[i]) return fail(YR_E_INVALID, "%s: null output %d", nm, i);
  int rc = check_program(program, n_words, n_in, n_out, gx, gy, gz, nm);
  if (rc != YR_OK) return rc;
  if (program[1] != dtype) return fail(YR_E_INVALID, "%s: program dtype", nm);
  Args a;
  memset(&a, 0, sizeof(a));
  for (int i = 0; i < n_in; i++) a.in[i] = (const uint16_t*)ins[i];
  for (int i = 0; i < n_out; i++) a.out[i] = (uint16_t*)outs[i];
  memcpy(a.w, program, sizeof(int32_t) * n_words);
  const size_t lds = (size_t)program[7];
  hipStream_t st = (hipStream_t)stream;
  const dim3 grid(gx, gy, gz);
  // more than 64 KiB of dynamic LDS needs the function's limit raised
  const void* fn = dtype == YR_DTYPE_BF16 ? (const void*)tb_program_kernel<DT_BF16> : (const void*)tb_program_kernel<DT_F16>;
  if (lds > 64 * 1024) {
    const hipError_t e = hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
    if (e != hipSuccess) return fail(YR_E_HIP, "%s: LDS limit %zu bytes: %s", nm, lds, hipGetErrorString(e));
  }
  if (dtype == YR_DTYPE_BF16) hipLaunchKernelGGL(tb_program_kernel<DT_BF16>, grid, dim3(kThreads), lds, st, a);
  else hipLaunchKernelGGL(tb_program_kernel<DT_F16>, grid, dim3(kThreads), lds, st, a);
  YR_CHECK_LAUNCH(nm);
  return YR_OK;
}

extern "C" int yr_hip_tb_program_check(const int32_t* program, int n_words, int n_in, int n_out, int gx, int gy,
                                       int gz) {
  if (!program) return yr::fail(YR_E_INVALID, "yr_hip_tb_program_check: null program");
  return yr::tbp::check_program(program, n_words, n_in, n_out, gx, gy, gz, "yr_hip_tb_program_check");
}
