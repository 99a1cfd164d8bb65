// Shared device/host helpers for the MI355X (gfx950, wave64) HIP backend.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>
#include <stddef.h>

#include "../../include/yirage_hip.h"

namespace yr {

constexpr int kWave = 64;

typedef _Float16 half_t;
typedef _Float16 half2v __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x2v __attribute__((ext_vector_type(2)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef __bf16 bf16x8v __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8v __attribute__((ext_vector_type(8)));

// ----------------------------------------------------------------- dtype tags
// DT_F16 / DT_BF16 select the 16-bit storage type; all math is fp32.
enum : int { DT_F16 = YR_DTYPE_F16, DT_BF16 = YR_DTYPE_BF16 };

// Workspace layout shared by every operator that needs one:
//   [0, kTicketBytes)  u32 arrival tickets, all zero at rest (each operator
//                      re-arms the tickets it used before it returns)
//   [kTicketBytes, ..) fp32 scratch (split partials), contents undefined
// A fixed ticket region means operators of different shapes can share one
// workspace without their scratch ever overlapping a ticket.
constexpr size_t kTicketBytes = 64 * 1024;
constexpr int kMaxTickets = (int)(kTicketBytes / 4);

__device__ __forceinline__ float bf16_bits_to_f32(uint32_t b16) {
  return __uint_as_float(b16 << 16);
}

// round-to-nearest-even f32 -> bf16 bits (v_cvt_pk_bf16_f32 on gfx950)
typedef __bf16 bf16x2_cvt __attribute__((ext_vector_type(2)));
__device__ __forceinline__ uint32_t f32x2_to_bf16x2_bits(float lo, float hi) {
  bf16x2_cvt v = {(__bf16)lo, (__bf16)hi};
  return __builtin_bit_cast(uint32_t, v);
}
__device__ __forceinline__ uint32_t f32_to_bf16_bits(float f) { return f32x2_to_bf16x2_bits(f, 0.f) & 0xffffu; }

__device__ __forceinline__ float f16_bits_to_f32(uint32_t h16) {
  union { uint16_t u; _Float16 h; } c;
  c.u = (uint16_t)h16;
  return (float)c.h;
}

__device__ __forceinline__ uint32_t f32_to_f16_bits(float f) {
  union { uint16_t u; _Float16 h; } c;
  c.h = (_Float16)f;  // v_cvt_f16_f32: round to nearest even
  return c.u;
}

template <int DT>
__device__ __forceinline__ float ld_elem(uint32_t bits16) {
  if constexpr (DT == DT_F16) return f16_bits_to_f32(bits16);
  else return bf16_bits_to_f32(bits16);
}

template <int DT>
__device__ __forceinline__ uint32_t st_elem(float v) {
  if constexpr (DT == DT_F16) return f32_to_f16_bits(v);
  else return f32_to_bf16_bits(v);
}

template <int DT>
__device__ __forceinline__ float round_to(float v) {
  return ld_elem<DT>(st_elem<DT>(v));
}

// low / high 16-bit element of a packed dword
template <int DT>
__device__ __forceinline__ float lo16(uint32_t w) { return ld_elem<DT>(w & 0xffffu); }
template <int DT>
__device__ __forceinline__ float hi16(uint32_t w) { return ld_elem<DT>(w >> 16); }

template <int DT>
__device__ __forceinline__ uint32_t pack2(float lo, float hi) {
  if constexpr (DT == DT_BF16) return f32x2_to_bf16x2_bits(lo, hi);
  else return st_elem<DT>(lo) | (st_elem<DT>(hi) << 16);
}

// fp32 += dot(a.xy, b.xy) on packed 16-bit pairs (v_dot2_f32_f16 / v_dot2_f32_bf16)
template <int DT>
__device__ __forceinline__ float dot2(uint32_t a, uint32_t b, float c) {
  if constexpr (DT == DT_F16) {
    half2v ha = __builtin_bit_cast(half2v, a);
    half2v hb = __builtin_bit_cast(half2v, b);
    return __builtin_amdgcn_fdot2(ha, hb, c, false);
  } else {
    bf16x2v ha = __builtin_bit_cast(bf16x2v, a);
    bf16x2v hb = __builtin_bit_cast(bf16x2v, b);
    return __builtin_amdgcn_fdot2_f32_bf16(ha, hb, c, false);
  }
}

// ----------------------------------------------------------------- wave ops
__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, kWave);
  return v;
}

// Max / sum over the 16 lanes of each 16-lane row (every lane of the row
// gets the result): DPP quad permutes and row mirrors, in registers.
__device__ __forceinline__ float dpp_f(float v, int ctrl_sel) {
  switch (ctrl_sel) {
    case 0: return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0xB1, 0xF, 0xF, false));
    case 1: return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0x4E, 0xF, 0xF, false));
    case 2: return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0x141, 0xF, 0xF, false));
    default: return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0x140, 0xF, 0xF, false));
  }
}
__device__ __forceinline__ float row16_max(float v) {
#pragma unroll
  for (int k = 0; k < 4; k++) v = fmaxf(v, dpp_f(v, k));
  return v;
}
__device__ __forceinline__ float row16_sum(float v) {
#pragma unroll
  for (int k = 0; k < 4; k++) v += dpp_f(v, k);
  return v;
}
// x + (x of lane l ^ 16) and x + (x of lane l ^ 32) by permlane swaps
__device__ __forceinline__ float add_xor16(float x) {
  const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}
__device__ __forceinline__ float add_xor32(float x) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

// Sum over the 64 lanes in registers: DPP within 16-lane rows, then the
// gfx950 permlane swaps across rows (no LDS round trips, unlike __shfl_xor).
__device__ __forceinline__ float wave_sum_regs(float v) {
  return add_xor32(add_xor16(row16_sum(v)));
}

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, kWave));
  return v;
}

// Global-memory pointers.  An access through a generic pointer compiles to a
// flat instruction, which counts against lgkmcnt as well as vmcnt: every
// later wait for an LDS or scalar result (lgkmcnt) then also waits for the
// flat access to come back through the CU's vector memory queue, which holds
// the whole weight prefetch (~1.7 us at 112 KiB in flight per CU, measured).
// Every device-memory access therefore goes through these casts, which
// make it a global_* instruction counted by vmcnt only.
#define YR_G __attribute__((address_space(1)))
template <class T>
__device__ __forceinline__ YR_G T* gptr(T* p) {
  return (YR_G T*)p;
}
template <class T>
__device__ __forceinline__ const YR_G T* gptr(const T* p) {
  return (const YR_G T*)p;
}

// (A plain cast of a uint4 pointer is not enough: copying the struct goes
// back through a generic pointer.  The accesses use a native vector type.)
typedef unsigned int yr_u32x4 __attribute__((ext_vector_type(4)));

// 128-bit global load that bypasses nothing special (cached); used for weights
__device__ __forceinline__ uint4 ldg16(const void* p) {
  return __builtin_bit_cast(uint4, *(const YR_G yr_u32x4*)p);
}

// 128-bit global store
__device__ __forceinline__ void stg16(void* p, uint4 v) {
  *(YR_G yr_u32x4*)p = __builtin_bit_cast(yr_u32x4, v);
}

// streaming (non-temporal) 128-bit load for data read exactly once
__device__ __forceinline__ uint4 ldg16_stream(const void* p) {
  return __builtin_bit_cast(uint4, __builtin_nontemporal_load((const YR_G yr_u32x4*)p));
}

// ---------------------------------------------------------------- cross-CU exchange
// Split-K style exchange between workgroups of one launch without cache
// maintenance: records are written with agent-scope (sc1) stores that go
// past the XCD-local L2, completion is awaited (vmcnt 0) before the arrival
// ticket is bumped, and the last arriving workgroup reads the records back
// with agent-scope (sc1) loads.  No buffer_wbl2 / buffer_inv is issued, which
// on gfx950 would walk the whole L2 of the XCD for every workgroup.
__device__ __forceinline__ void st_agent(float* p, float v) {
  __hip_atomic_store((YR_G uint32_t*)p, __float_as_uint(v), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

__device__ __forceinline__ void st_agent4(float* p, float4 v) {
  uint64_t lo = (uint64_t)__float_as_uint(v.x) | ((uint64_t)__float_as_uint(v.y) << 32);
  uint64_t hi = (uint64_t)__float_as_uint(v.z) | ((uint64_t)__float_as_uint(v.w) << 32);
  __hip_atomic_store((YR_G uint64_t*)p, lo, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  __hip_atomic_store((YR_G uint64_t*)p + 1, hi, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

__device__ __forceinline__ float ld_agent(const float* p) {
  return __uint_as_float(__hip_atomic_load((const YR_G uint32_t*)p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT));
}

__device__ __forceinline__ float4 ld_agent4(const float* p) {
  uint64_t lo = __hip_atomic_load((const YR_G uint64_t*)p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  uint64_t hi = __hip_atomic_load((const YR_G uint64_t*)p + 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  return make_float4(__uint_as_float((uint32_t)lo), __uint_as_float((uint32_t)(lo >> 32)),
                     __uint_as_float((uint32_t)hi), __uint_as_float((uint32_t)(hi >> 32)));
}

__device__ __forceinline__ void wait_vm() { __builtin_amdgcn_s_waitcnt(0); }

// Copy n floats (n % 4 == 0) from LDS to a record with agent-scope stores.
__device__ __forceinline__ void put_record(float* rec, const float* src, int n) {
  for (int i = threadIdx.x * 4; i < n; i += blockDim.x * 4)
    st_agent4(rec + i, make_float4(src[i], src[i + 1], src[i + 2], src[i + 3]));
}

// Every thread's agent stores complete, then one arrival on *ticket.
// Returns true in every thread of the workgroup that arrived last (of n);
// that workgroup re-arms the ticket to 0.
__device__ __forceinline__ bool arrive_last(uint32_t* ticket, int n) {
  __shared__ int s_last;
  wait_vm();
  __syncthreads();
  if (threadIdx.x == 0) {
    uint32_t old = __hip_atomic_fetch_add(gptr(ticket), 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    s_last = old == (uint32_t)(n - 1);
    if (s_last) __hip_atomic_store(gptr(ticket), 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
  __syncthreads();
  return s_last != 0;
}

// Sum S records of `rec` floats (rec % 4 == 0) laid out back to back at
// `base` into dst[0..rec), in record order s = 0..S-1 (deterministic).  Each
// thread keeps up to 8 independent 16-byte loads in flight, so the S records
// cost ceil(S / 8) memory round trips instead of S.
__device__ __forceinline__ void sum_records(const float* base, int S, int rec, float* dst) {
  for (int i = threadIdx.x * 4; i < rec; i += blockDim.x * 4) {
    float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
    int s = 0;
    for (; s + 8 <= S; s += 8) {
      float4 v[8];
#pragma unroll
      for (int u = 0; u < 8; u++) v[u] = ld_agent4(base + (size_t)(s + u) * rec + i);
#pragma unroll
      for (int u = 0; u < 8; u++) {
        acc.x += v[u].x; acc.y += v[u].y; acc.z += v[u].z; acc.w += v[u].w;
      }
    }
    for (; s < S; s++) {
      float4 v = ld_agent4(base + (size_t)s * rec + i);
      acc.x += v.x; acc.y += v.y; acc.z += v.z; acc.w += v.w;
    }
    dst[i] = acc.x; dst[i + 1] = acc.y; dst[i + 2] = acc.z; dst[i + 3] = acc.w;
  }
}

// ---------------------------------------------------------------- MFMA operands
// ds_read_b64_tr_b16: within a 16-lane group, lane i element e of the result
// is element i % 4 of the 64-bit row that lane 4e + i / 4 addressed.
typedef short v4i16 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) v4i16 lds_v4i16;

// B fragment of a 32 x 16 block of a row-major [rows][ld] bf16/f16 tile in
// LDS whose first row is `row0`.
__device__ __forceinline__ uint4 b_frag(const uint16_t* tile, int ld, int row0, int lane) {
  const int g = lane >> 4, j = lane & 15, e = j >> 2, q = j & 3;
  const uint16_t* p0 = tile + (row0 + 8 * g + e) * ld + 4 * q;
  const uint16_t* p1 = p0 + 4 * ld;
  auto cast = [](const uint16_t* p) __attribute__((always_inline)) {
    return reinterpret_cast<const lds_v4i16*>(
        reinterpret_cast<const __attribute__((address_space(3))) uint16_t*>(
            reinterpret_cast<uintptr_t>(p)));
  };
  const v4i16 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16(const_cast<lds_v4i16*>(cast(p0)));
  const v4i16 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16(const_cast<lds_v4i16*>(cast(p1)));
  const uint2 l2 = __builtin_bit_cast(uint2, lo), h2 = __builtin_bit_cast(uint2, hi);
  return make_uint4(l2.x, l2.y, h2.x, h2.y);
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

__host__ __device__ constexpr int round_up4(int x) { return (x + 3) & ~3; }

__device__ __forceinline__ float silu(float a) { return a / (1.0f + __expf(-a)); }

}  // namespace yr

// ----------------------------------------------------------------- host side
namespace yr {
void set_error(const char* fmt, ...);
int fail(int code, const char* fmt, ...);
int check_hip(hipError_t e, const char* what);
}  // namespace yr

#define YR_CHECK_LAUNCH(what)                                    \
  do {                                                           \
    hipError_t _e = hipGetLastError();                           \
    if (_e != hipSuccess) return yr::check_hip(_e, what);        \
  } while (0)
