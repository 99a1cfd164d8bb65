// Bandwidth-bound skinny GEMMs for gfx950 with the weight in N x K layout
// (W[N][K], torch Linear.weight): RMSNorm+linear, gated MLP and
// linear(+residual) for passes of up to 8 rows.  (K x N weights, and N x K
// passes of more than 16 rows, run on the MFMA kernels of skinny.hip.)
//
// Design:
//  * Weights stream once from HBM with 128-bit loads; every lane issues all of
//    its weight loads before it touches the activations, so the whole tile is
//    in flight while X is staged and the norm statistic is formed.
//  * Inner products use v_dot2_f32_{f16,bf16} (two MACs per lane-op, fp32
//    accumulate) over contiguous K chunks of a weight row.
//  * The K dimension is split across workgroups so the grid fills all 256
//    CUs; each workgroup reduces its waves in LDS, writes one fp32 partial
//    record, and the last workgroup to arrive for an output tile (atomic
//    ticket) sums the records in a fixed order and applies the epilogue
//    (RMS scale / SiLU-mul / residual / rounding).  Deterministic, one launch.
#include <stdarg.h>
#include <stdio.h>

#include "yr_common.h"

namespace yr {

// K x N weights go to the MFMA kernels of skinny.hip
size_t skinny_kn_workspace(int B, int K, int N, int nmat, int epi);
int skinny_kn(const uint16_t* x, const uint16_t* gamma, const uint16_t* w0, const uint16_t* w1,
              const uint16_t* residual, uint16_t* out, int B, int K, int N, float eps, int dtype, int nmat, int epi,
              void* ws, size_t ws_bytes, hipStream_t st, const char* name);
// N x K weights, passes of 17..128 rows: the MFMA kernel of skinny.hip
size_t skinny_nk128_workspace(int K, int N, int nmat, int epi);
int skinny_nk128(const uint16_t* x, const uint16_t* gamma, const uint16_t* w0, const uint16_t* w1,
                 const uint16_t* residual, uint16_t* out, int B, int K, int N, float eps, int dtype, int nmat,
                 int epi, void* ws, hipStream_t st, const char* name);

enum : int { EPI_LINEAR = 0, EPI_RMSNORM = 1, EPI_GATED = 2 };

struct GemvArgs {
  const uint16_t* x;        // [B][K]
  const uint16_t* gamma;    // [K] or null
  const uint16_t* w0;       // weights (W or W1)
  const uint16_t* w1;       // W3 for the gated MLP
  const uint16_t* residual; // [B][N] or null
  uint16_t* out;            // [B][N]
  float* partial;           // [tiles][S][rec]
  uint32_t* tickets;        // [tiles]
  int B, K, N, S;           // S: number of K splits
  int ldx, ldo;             // row strides of x / out (elements)
  float eps;
};

// ---------------------------------------------------------------- NK layout
// W[N][K] row-major (torch Linear.weight).  A lane owns C 16-byte chunks of
// the K slice (chunk lane + 64*c) and keeps the matching x chunks of all NB
// batch rows in registers; a wave walks output rows, four at a time, so 4*C
// weight loads per lane are in flight.  Per-row lane reduction uses a
// reduce-scatter over the NB values (10 shuffles for NB = 8, not 48).
// Workgroup tile: NK_ROWS output rows x (64 * 8 * C) K elements.
constexpr int NK_WAVES = 8;
constexpr int NK_THREADS = NK_WAVES * kWave;

template <int NB>
__device__ __forceinline__ void wave_reduce_nb(float (&v)[NB], int lane) {
  // full butterfly for small NB
#pragma unroll
  for (int b = 0; b < NB; b++) v[b] = wave_sum(v[b]);
  (void)lane;
}

template <int DT, int NB, int NMAT, int EPI, int C, int TROWS>
__global__ __launch_bounds__(NK_THREADS) void gemv_nk_kernel(GemvArgs a) {
  constexpr int KS = kWave * 8 * C;  // K elements per workgroup
  __shared__ float red[round_up4(NMAT * NB * TROWS + NB)];
  __shared__ float ssl[NK_WAVES];

  const int tid = threadIdx.x;
  const int wave = tid / kWave, lane = tid % kWave;
  const int tile = blockIdx.x, split = blockIdx.y;
  const int n_base = tile * TROWS;
  const int k0 = split * KS;

  // x chunks of this lane for all batch rows (gamma applied), kept in VGPRs
  uint32_t xr[NB][C][4];
  float ss_part = 0.f;
#pragma unroll
  for (int c = 0; c < C; c++) {
    int k = k0 + (lane + kWave * c) * 8;
    uint4 gv = make_uint4(0, 0, 0, 0);
    bool kok = k < a.K;
    if constexpr (EPI == EPI_RMSNORM)
      if (a.gamma && kok) gv = ldg16(a.gamma + k);
    uint32_t gw[4] = {gv.x, gv.y, gv.z, gv.w};
#pragma unroll
    for (int b = 0; b < NB; b++) {
      uint4 xv = make_uint4(0, 0, 0, 0);
      if (kok && b < a.B) xv = ldg16(a.x + (size_t)b * a.ldx + k);
      uint32_t xw[4] = {xv.x, xv.y, xv.z, xv.w};
#pragma unroll
      for (int j = 0; j < 4; j++) {
        float lo = lo16<DT>(xw[j]), hi = hi16<DT>(xw[j]);
        if (b == wave % NB && wave < NB) ss_part += lo * lo + hi * hi;
        uint32_t p = xw[j];
        if constexpr (EPI == EPI_RMSNORM)
          if (a.gamma) p = pack2<DT>(lo * lo16<DT>(gw[j]), hi * hi16<DT>(gw[j]));
        xr[b][c][j] = p;
      }
    }
  }
  if constexpr (EPI == EPI_RMSNORM) {
    float s = wave_sum(ss_part);
    if (lane == 0) ssl[wave] = s;
  }

  // rows of this wave: wave, wave + 8, ... (TROWS / NK_WAVES rows), 4 at a time
  constexpr int RPWV = TROWS / NK_WAVES;
  constexpr int RU = RPWV < 4 ? RPWV : 4;
#pragma unroll 1
  for (int r0 = 0; r0 < RPWV; r0 += RU) {
    uint4 w[NMAT][RU][C];
#pragma unroll
    for (int m = 0; m < NMAT; m++) {
      const uint16_t* W = m == 0 ? a.w0 : a.w1;
#pragma unroll
      for (int u = 0; u < RU; u++) {
        int n = n_base + wave + NK_WAVES * (r0 + u);
#pragma unroll
        for (int c = 0; c < C; c++) {
          int k = k0 + (lane + kWave * c) * 8;
          if (n < a.N && k < a.K) w[m][u][c] = ldg16(W + (size_t)n * a.K + k);
          else w[m][u][c] = make_uint4(0, 0, 0, 0);
        }
      }
    }
#pragma unroll
    for (int m = 0; m < NMAT; m++)
#pragma unroll
      for (int u = 0; u < RU; u++) {
        float v[NB];
#pragma unroll
        for (int b = 0; b < NB; b++) {
          float s = 0.f;
#pragma unroll
          for (int c = 0; c < C; c++) {
            s = dot2<DT>(w[m][u][c].x, xr[b][c][0], s);
            s = dot2<DT>(w[m][u][c].y, xr[b][c][1], s);
            s = dot2<DT>(w[m][u][c].z, xr[b][c][2], s);
            s = dot2<DT>(w[m][u][c].w, xr[b][c][3], s);
          }
          v[b] = s;
        }
        wave_reduce_nb<NB>(v, lane);
        if (lane == 0) {
          int rl = wave + NK_WAVES * (r0 + u);
#pragma unroll
          for (int b = 0; b < NB; b++) red[(m * NB + b) * TROWS + rl] = v[b];
        }
      }
  }
  __syncthreads();
  if (tid < NB) {
    float s = 0.f;
    if constexpr (EPI == EPI_RMSNORM) s = ssl[tid];
    red[NMAT * NB * TROWS + tid] = s;
  }
  __syncthreads();

  // split-K combine (same ticket protocol as the KN kernel, tile width TROWS)
  constexpr int REC = round_up4(NMAT * NB * TROWS + NB);
  const float* fin = red;
  __shared__ float sum[REC];
  if (a.S > 1) {
    put_record(a.partial + ((size_t)tile * a.S + split) * REC, red, REC);
    if (!arrive_last(&a.tickets[tile], a.S)) return;
    sum_records(a.partial + (size_t)tile * a.S * REC, a.S, REC, sum);
    __syncthreads();
    fin = sum;
  }
  for (int i = tid; i < NB * TROWS; i += NK_THREADS) {
    int b = i / TROWS, rl = i % TROWS, n = n_base + rl;
    if (b >= a.B || n >= a.N) continue;
    float v = fin[b * TROWS + rl];
    if constexpr (EPI == EPI_RMSNORM) {
      v *= rsqrtf(fin[NMAT * NB * TROWS + b] / (float)a.K + a.eps);
    } else if constexpr (EPI == EPI_GATED) {
      v = silu(v) * fin[(NB + b) * TROWS + rl];
    }
    if (a.residual) v += ld_elem<DT>(a.residual[(size_t)b * a.ldo + n]);
    a.out[(size_t)b * a.ldo + n] = (uint16_t)st_elem<DT>(v);
  }
}

// ---------------------------------------------------------------- host side
constexpr int NK_C1 = 4;       // 16-byte chunks per lane per row, batch 1 (K slice 2048)
constexpr int NK_C8 = 2;       // same for batch 2..8 (x of 8 rows stays in VGPRs)
constexpr int NK_TROWS = 32;   // output rows per workgroup

struct Plan {
  int tiles, S, rec;
  size_t ws;
};


static Plan plan_gemv(int B, int K, int N, int nmat) {
  Plan p;
  const int nb = 8;
  const int ks = kWave * 8 * (B == 1 ? NK_C1 : NK_C8);
  p.tiles = (N + NK_TROWS - 1) / NK_TROWS;
  p.S = (K + ks - 1) / ks;
  p.rec = round_up4(nmat * nb * NK_TROWS + nb);
  p.ws = 0;
  if (p.S > 1) p.ws = kTicketBytes + (size_t)p.tiles * p.S * p.rec * sizeof(float);
  return p;
}

template <int DT, int NMAT, int EPI>
static void launch_nk(const GemvArgs& a, hipStream_t st) {
  dim3 grid((a.N + NK_TROWS - 1) / NK_TROWS, a.S);
  if (a.B == 1)
    hipLaunchKernelGGL((gemv_nk_kernel<DT, 1, NMAT, EPI, NK_C1, NK_TROWS>), grid, dim3(NK_THREADS), 0, st, a);
  else
    hipLaunchKernelGGL((gemv_nk_kernel<DT, 8, NMAT, EPI, NK_C8, NK_TROWS>), grid, dim3(NK_THREADS), 0, st, a);
}

// Rows of the pass starting with `left` rows to go: up to 128 on the MFMA
// kernel while more than 16 remain, then chunks of up to 8 on the GEMV (each
// pass streams the weights once).
static int pass_rows(int left) { return left > 16 ? (left < 128 ? left : 128) : (left < 8 ? left : 8); }

static size_t nk_workspace(int B, int K, int N, int nmat, int epi) {
  size_t need = 0;
  for (int b0 = 0; b0 < B; b0 += pass_rows(B - b0)) {
    const int rows = pass_rows(B - b0);
    const size_t w = rows > 16 ? skinny_nk128_workspace(K, N, nmat, epi) : plan_gemv(rows, K, N, nmat).ws;
    if (w > need) need = w;
  }
  return need;
}

template <int NMAT, int EPI>
static int run_gemv(GemvArgs a, int dtype, int layout, void* ws, size_t ws_bytes, hipStream_t st,
                    const char* name) {
  if (a.B <= 0 || a.K <= 0 || a.N <= 0) return fail(YR_E_INVALID, "%s: empty shape", name);
  if (a.K % 8 || a.N % 8) return fail(YR_E_INVALID, "%s: K and N must be multiples of 8 (K=%d N=%d)", name, a.K, a.N);
  if (dtype != YR_DTYPE_F16 && dtype != YR_DTYPE_BF16) return fail(YR_E_INVALID, "%s: dtype must be f16/bf16", name);
  if (layout != YR_W_KN && layout != YR_W_NK) return fail(YR_E_INVALID, "%s: bad weight layout", name);
  if (!a.x || !a.w0 || !a.out || (NMAT == 2 && !a.w1)) return fail(YR_E_INVALID, "%s: null pointer", name);
  if (layout == YR_W_KN)
    return skinny_kn(a.x, a.gamma, a.w0, a.w1, a.residual, a.out, a.B, a.K, a.N, a.eps, dtype, NMAT, EPI, ws,
                     ws_bytes, st, name);
  const size_t need = nk_workspace(a.B, a.K, a.N, NMAT, EPI);
  if (need > ws_bytes || (need && !ws))
    return fail(YR_E_WORKSPACE, "%s: workspace %zu < required %zu", name, ws_bytes, need);
  {
    Plan q = plan_gemv(a.B < 8 ? a.B : 8, a.K, a.N, NMAT);
    if (q.tiles > kMaxTickets) return fail(YR_E_INVALID, "%s: N=%d too large (%d tiles)", name, a.N, q.tiles);
  }
  a.ldx = a.K;
  a.ldo = a.N;
  const int B = a.B;
  for (int b0 = 0; b0 < B; b0 += pass_rows(B - b0)) {
    GemvArgs c = a;
    c.B = pass_rows(B - b0);
    c.x = a.x + (size_t)b0 * a.K;
    c.out = a.out + (size_t)b0 * a.N;
    if (a.residual) c.residual = a.residual + (size_t)b0 * a.N;
    if (c.B > 16) {
      const int rc = skinny_nk128(c.x, c.gamma, c.w0, c.w1, c.residual, c.out, c.B, a.K, a.N, a.eps, dtype, NMAT,
                                  EPI, ws, st, name);
      if (rc != YR_OK) return rc;
      continue;
    }
    Plan p = plan_gemv(c.B, a.K, a.N, NMAT);
    c.S = p.S;
    if (p.ws) {
      c.tickets = (uint32_t*)ws;
      c.partial = (float*)((char*)ws + kTicketBytes);
    }
    if (dtype == YR_DTYPE_F16) launch_nk<DT_F16, NMAT, EPI>(c, st);
    else launch_nk<DT_BF16, NMAT, EPI>(c, st);
    YR_CHECK_LAUNCH(name);
  }
  return YR_OK;
}

}  // namespace yr

using namespace yr;

extern "C" {

static size_t ws_for(int batch, int k, int n, int w_layout, int nmat, int epi) {
  if (w_layout == YR_W_KN) return skinny_kn_workspace(batch, k, n, nmat, epi);
  return nk_workspace(batch, k, n, nmat, epi);
}

size_t yr_hip_rmsnorm_linear_workspace(int batch, int k, int n, int dtype, int w_layout) {
  (void)dtype;
  return ws_for(batch, k, n, w_layout, 1, EPI_RMSNORM);
}

size_t yr_hip_gated_mlp_workspace(int batch, int k, int n, int dtype, int w_layout) {
  (void)dtype;
  return ws_for(batch, k, n, w_layout, 2, EPI_GATED);
}

size_t yr_hip_linear_workspace(int batch, int k, int n, int dtype, int w_layout) {
  (void)dtype;
  return ws_for(batch, k, n, w_layout, 1, EPI_LINEAR);
}

int yr_hip_rmsnorm_linear(const void* x, const void* gamma, const void* w, void* out, int batch, int k,
                          int n, int dtype, int w_layout, float eps, void* workspace,
                          size_t workspace_bytes, void* stream) {
  GemvArgs a = {};
  a.x = (const uint16_t*)x;
  a.gamma = (const uint16_t*)gamma;
  a.w0 = (const uint16_t*)w;
  a.out = (uint16_t*)out;
  a.B = batch; a.K = k; a.N = n; a.eps = eps;
  return run_gemv<1, EPI_RMSNORM>(a, dtype, w_layout, workspace, workspace_bytes, (hipStream_t)stream,
                                   "yr_hip_rmsnorm_linear");
}

int yr_hip_gated_mlp(const void* x, const void* w1, const void* w3, void* out, int batch, int k, int n,
                     int dtype, int w_layout, void* workspace, size_t workspace_bytes, void* stream) {
  GemvArgs a = {};
  a.x = (const uint16_t*)x;
  a.w0 = (const uint16_t*)w1;
  a.w1 = (const uint16_t*)w3;
  a.out = (uint16_t*)out;
  a.B = batch; a.K = k; a.N = n;
  return run_gemv<2, EPI_GATED>(a, dtype, w_layout, workspace, workspace_bytes, (hipStream_t)stream,
                                 "yr_hip_gated_mlp");
}

int yr_hip_linear(const void* x, const void* w, const void* residual, void* out, int batch, int k,
                  int n, int dtype, int w_layout, void* workspace, size_t workspace_bytes,
                  void* stream) {
  GemvArgs a = {};
  a.x = (const uint16_t*)x;
  a.w0 = (const uint16_t*)w;
  a.residual = (const uint16_t*)residual;
  a.out = (uint16_t*)out;
  a.B = batch; a.K = k; a.N = n;
  return run_gemv<1, EPI_LINEAR>(a, dtype, w_layout, workspace, workspace_bytes, (hipStream_t)stream,
                                  "yr_hip_linear");
}

}  // extern "C"
