// Error reporting, device queries and the deterministic synthetic-data
// generator of the hip backend.
#include <stdarg.h>
#include <stdio.h>
#include <string.h>

#include "yr_common.h"

namespace yr {

static thread_local char g_err[1024] = "";

void set_error(const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof(g_err), fmt, ap);
  va_end(ap);
}

int fail(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof(g_err), fmt, ap);
  va_end(ap);
  return code;
}

int check_hip(hipError_t e, const char* what) {
  if (e == hipSuccess) return YR_OK;
  return fail(YR_E_HIP, "%s: HIP error %d (%s)", what, (int)e, hipGetErrorString(e));
}

// ------------------------------------------------------------ synthetic data
// splitmix64 finaliser; must stay bit-identical to the CPU generator.
__device__ __forceinline__ uint64_t mix64(uint64_t x) {
  x += 0x9E3779B97F4A7C15ull;
  x = (x ^ (x >> 30)) * 0xBF58476D1CE4E5B9ull;
  x = (x ^ (x >> 27)) * 0x94D049BB133111EBull;
  return x ^ (x >> 31);
}

// f32 -> f16 bits, round to nearest even, in integer arithmetic so that the
// compiler cannot fold the preceding multiply into a single-rounding
// v_fma_mix (the CPU generator rounds the product to f32 first).
__device__ __forceinline__ uint32_t f32_to_f16_bits_int(float f) {
  uint32_t u = __float_as_uint(f);
  uint32_t sign = (u >> 16) & 0x8000u, a = u & 0x7fffffffu;
  if (a > 0x7f800000u) return sign | 0x7e00u;
  if (a >= 0x477ff000u) return sign | 0x7c00u;
  if (a < 0x38800000u) {  // f16 subnormal range: value / 2^-24, ties to even
    uint32_t e = a >> 23, m = (a & 0x7fffffu) | 0x800000u;
    int shift = 126 - (int)e;  // bits to drop so the unit is 2^-24
    if (shift > 24) return sign;
    uint32_t q = m >> shift, rem = m & ((1u << shift) - 1u), half = 1u << (shift - 1);
    if (rem > half || (rem == half && (q & 1u))) q++;
    return sign | q;
  }
  uint32_t h = ((((a >> 23) - 112u) << 10) | ((a & 0x7fffffu) >> 13));
  uint32_t rem = a & 0x1fffu;
  if (rem > 0x1000u || (rem == 0x1000u && (h & 1u))) h++;
  return sign | h;
}

template <int DT>
__global__ void synth_fill_kernel(uint16_t* dst, size_t n, uint64_t seed_mixed, uint64_t offset, float scale) {
  size_t stride = (size_t)gridDim.x * blockDim.x;
  for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride) {
    uint64_t h = mix64(seed_mixed ^ ((offset + i) * 0xD1342543DE82EF95ull));
    int32_t s = (int32_t)(h & 0xffff) + (int32_t)((h >> 16) & 0xffff) + (int32_t)((h >> 32) & 0xffff) +
                (int32_t)((h >> 48) & 0xffff) - 131070;
    float v = (float)s * scale;
    dst[i] = (uint16_t)(DT == DT_F16 ? f32_to_f16_bits_int(v) : f32_to_bf16_bits(v));
  }
}

static uint64_t host_mix64(uint64_t x) {
  x += 0x9E3779B97F4A7C15ull;
  x = (x ^ (x >> 30)) * 0xBF58476D1CE4E5B9ull;
  x = (x ^ (x >> 27)) * 0x94D049BB133111EBull;
  return x ^ (x >> 31);
}

}  // namespace yr

using namespace yr;

extern "C" {

const char* yr_hip_last_error(void) { return g_err; }

const char* yr_hip_version(void) { return "yirage-hip 0.1.0 (gfx950)"; }

int yr_hip_device_info(int device_id, yr_device_info* out) {
  if (!out) return fail(YR_E_INVALID, "yr_hip_device_info: null output");
  int count = 0;
  hipError_t e = hipGetDeviceCount(&count);
  if (e != hipSuccess || count == 0) return fail(YR_E_NODEVICE, "no HIP device visible");
  if (device_id < 0 || device_id >= count) return fail(YR_E_INVALID, "device %d out of range", device_id);
  hipDeviceProp_t p;
  e = hipGetDeviceProperties(&p, device_id);
  if (e != hipSuccess) return check_hip(e, "hipGetDeviceProperties");
  memset(out, 0, sizeof(*out));
  out->device_id = device_id;
  out->num_compute_units = p.multiProcessorCount;
  out->compute_capability = p.major * 100 + p.minor * 10;  // gfx950 -> 9,5 -> 950
  out->wavefront_size = p.warpSize;
  out->total_memory = p.totalGlobalMem;
  out->max_shared_memory = p.sharedMemPerBlock;
  out->clock_khz = p.clockRate;
  strncpy(out->arch_name, p.gcnArchName, sizeof(out->arch_name) - 1);
  return YR_OK;
}

int yr_hip_synth_fill(void* dst, size_t n, int dtype, uint64_t seed, uint64_t offset, float stddev,
                      void* stream) {
  if (!dst && n) return fail(YR_E_INVALID, "yr_hip_synth_fill: null destination");
  if (n == 0) return YR_OK;
  float scale = stddev / 37837.2265f;
  uint64_t sm = host_mix64(seed);
  size_t blocks = (n + 255) / 256;
  if (blocks > 65536) blocks = 65536;
  hipStream_t st = (hipStream_t)stream;
  if (dtype == YR_DTYPE_BF16)
    hipLaunchKernelGGL(synth_fill_kernel<DT_BF16>, dim3((unsigned)blocks), dim3(256), 0, st, (uint16_t*)dst, n, sm, offset, scale);
  else if (dtype == YR_DTYPE_F16)
    hipLaunchKernelGGL(synth_fill_kernel<DT_F16>, dim3((unsigned)blocks), dim3(256), 0, st, (uint16_t*)dst, n, sm, offset, scale);
  else
    return fail(YR_E_INVALID, "yr_hip_synth_fill: dtype must be f16/bf16");
  YR_CHECK_LAUNCH("yr_hip_synth_fill");
  return YR_OK;
}

}  // extern "C"
