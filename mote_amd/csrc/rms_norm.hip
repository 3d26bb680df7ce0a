// Fused residual add + RMSNorm, forward and backward (the RMSNorm of mote/model/norm.py:26-59, the
// pre-norm of every H-Net block, blocks.py:37, 50, and the final norm, :95).
//
// Forward, per row of D elements (everything in fp32):
//   s = x + residual           (residual given; residual_in_fp32: both upcast first)
//   r = 1 / sqrt(mean(s^2) + eps)
//   y = (s r w) in the dtype of x; the new residual stream is s (fp32 when residual_in_fp32)
// Backward, with g = dy w and the saved s and r:
//   ds = r g - (r^3 / D) s sum(g s) + dres_out      (dres_out: gradient of the returned residual)
//   dx = ds (dtype of x), dresidual = ds (dtype of the residual), dw = sum over rows of dy s r
// dw is summed deterministically: one fp32 partial per workgroup and element, then a fixed-order sum.
//
// One wave per row: lane l owns the 4-element units l, l + 64, ... (NU units, D <= 256 NU), so a row
// is read and written in 8-byte (bf16) or 16-byte (fp32) pieces that are contiguous across the wave.
// HBM-bound by design: no LDS in the forward; in the backward an LDS reduction of the dw sums per
// workgroup (at most 256 workgroups) and a second kernel that adds the partials in a fixed order.
#include "common.hpp"
#include "params.hpp"

namespace mote {

struct NormParams {
  const void* x; int64_t x_sr;
  const void* res; int64_t r_sr;      // null: no residual
  const float* w;
  void* y; int64_t y_sr;
  void* res_out; int64_t ro_sr;       // null: the sum is not returned
  float* rstd;                        // null: not saved
  int rows, D, x_f32, res_f32, out_f32, res_out_f32;
  int round_sum;                      // the sum stream is bf16: round s before the norm
  float eps;
};

struct NormBwdParams {
  const void* dy; int64_t dy_sr;
  const void* dro; int64_t dro_sr;    // null: no gradient for the returned residual
  const void* s; int64_t s_sr;        // the saved sum
  const float* rstd;
  const float* w;
  void* dx; int64_t dx_sr;
  void* dres; int64_t dres_sr;        // null: no residual input
  float* part;                        // [gridDim.x][D] dw partials
  float* dw;
  int rows, D, dy_f32, dro_f32, s_f32, dx_f32, dres_f32;
};

constexpr int kNormWaves = 4;        // forward: rows per workgroup (one wave each)
constexpr int kNormBwdBlocks = 256;  // backward: at most one workgroup per CU, so at most 256 dw partials
constexpr int kNormDwWaves = 16;     // dw sum: waves per 64-element strip

// 4 consecutive elements of a row as fp32: from fp32 (16 bytes) or bf16 (8 bytes) memory
__device__ __forceinline__ void load4(const void* base, int64_t off, bool f32, float (&v)[4]) {
  if (f32) {
    const float4 a = *reinterpret_cast<const float4*>(reinterpret_cast<const float*>(base) + off);
    v[0] = a.x; v[1] = a.y; v[2] = a.z; v[3] = a.w;
  } else {
    const uint2 a = *reinterpret_cast<const uint2*>(reinterpret_cast<const bf16_t*>(base) + off);
    v[0] = bf2f(a.x & 0xffffu); v[1] = bf2f(a.x >> 16); v[2] = bf2f(a.y & 0xffffu); v[3] = bf2f(a.y >> 16);
  }
}
__device__ __forceinline__ void store4(void* base, int64_t off, bool f32, const float (&v)[4]) {
  if (f32) {
    *reinterpret_cast<float4*>(reinterpret_cast<float*>(base) + off) = make_float4(v[0], v[1], v[2], v[3]);
  } else {
    uint2 a;
    a.x = uint32_t(f2bf(v[0])) | (uint32_t(f2bf(v[1])) << 16);
    a.y = uint32_t(f2bf(v[2])) | (uint32_t(f2bf(v[3])) << 16);
    *reinterpret_cast<uint2*>(reinterpret_cast<bf16_t*>(base) + off) = a;
  }
}
__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) v += __shfl_xor(v, m, 64);
  return v;
}

template <int NU>
__global__ void __launch_bounds__(64 * kNormWaves) add_rms_norm_fwd_kernel(const NormParams p) {
  const int lane = threadIdx.x & 63;
  const int row = blockIdx.x * kNormWaves + (threadIdx.x >> 6);
  if (row >= p.rows) return;
  const int nu = p.D / 4;
  float s[NU][4];
  // loads first (units past the row read unit 0 again; their values are not used)
#pragma unroll
  for (int k = 0; k < NU; ++k) {
    const int u = min(lane + 64 * k, nu - 1);
    load4(p.x, int64_t(row) * p.x_sr + 4 * u, p.x_f32, s[k]);
  }
  if (p.res) {
    float r[NU][4];
#pragma unroll
    for (int k = 0; k < NU; ++k) {
      const int u = min(lane + 64 * k, nu - 1);
      load4(p.res, int64_t(row) * p.r_sr + 4 * u, p.res_f32, r[k]);
    }
#pragma unroll
    for (int k = 0; k < NU; ++k)
#pragma unroll
      for (int e = 0; e < 4; ++e) s[k][e] = p.round_sum ? bf2f(f2bf(s[k][e] + r[k][e])) : s[k][e] + r[k][e];
  }
  float ss = 0.f;
#pragma unroll
  for (int k = 0; k < NU; ++k)
    if (lane + 64 * k < nu)
#pragma unroll
      for (int e = 0; e < 4; ++e) ss = fmaf(s[k][e], s[k][e], ss);
  ss = wave_sum(ss);
  const float rs = 1.0f / sqrtf(ss / float(p.D) + p.eps);
#pragma unroll
  for (int k = 0; k < NU; ++k) {
    const int u = lane + 64 * k;
    if (u >= nu) continue;
    const float4 w4 = *reinterpret_cast<const float4*>(p.w + 4 * u);
    const float wv[4] = {w4.x, w4.y, w4.z, w4.w};
    float yv[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) yv[e] = s[k][e] * rs * wv[e];
    store4(p.y, int64_t(row) * p.y_sr + 4 * u, p.out_f32, yv);
    if (p.res_out) store4(p.res_out, int64_t(row) * p.ro_sr + 4 * u, p.res_out_f32, s[k]);
  }
  if (p.rstd && lane == 0) p.rstd[row] = rs;
}

// Each workgroup of NW waves walks rows blockIdx.x * NW + wave, + gridDim.x * NW, ...; a lane keeps its
// elements' dw sums in registers, the waves add them through LDS in a fixed order.
template <int NU, int NW>
__global__ void __launch_bounds__(64 * NW) add_rms_norm_bwd_kernel(const NormBwdParams p) {
  __shared__ __align__(16) float red[NW][NU * 256];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int nu = p.D / 4;
  float dwacc[NU][4];
#pragma unroll
  for (int k = 0; k < NU; ++k)
#pragma unroll
    for (int e = 0; e < 4; ++e) dwacc[k][e] = 0.f;
  float wv[NU][4];
#pragma unroll
  for (int k = 0; k < NU; ++k) {
    const int u = min(lane + 64 * k, nu - 1);
    const float4 w4 = *reinterpret_cast<const float4*>(p.w + 4 * u);
    wv[k][0] = w4.x; wv[k][1] = w4.y; wv[k][2] = w4.z; wv[k][3] = w4.w;
  }
  for (int row = blockIdx.x * NW + wave; row < p.rows; row += gridDim.x * NW) {
    float dy[NU][4], s[NU][4], dro[NU][4];
#pragma unroll
    for (int k = 0; k < NU; ++k) {
      const int u = min(lane + 64 * k, nu - 1);
      load4(p.dy, int64_t(row) * p.dy_sr + 4 * u, p.dy_f32, dy[k]);
      load4(p.s, int64_t(row) * p.s_sr + 4 * u, p.s_f32, s[k]);
    }
    if (p.dro) {
#pragma unroll
      for (int k = 0; k < NU; ++k) {
        const int u = min(lane + 64 * k, nu - 1);
        load4(p.dro, int64_t(row) * p.dro_sr + 4 * u, p.dro_f32, dro[k]);
      }
    }
    const float rs = p.rstd[row];
    float gs = 0.f;
#pragma unroll
    for (int k = 0; k < NU; ++k)
      if (lane + 64 * k < nu)
#pragma unroll
        for (int e = 0; e < 4; ++e) gs = fmaf(dy[k][e] * wv[k][e], s[k][e], gs);
    gs = wave_sum(gs);
    const float c = rs * rs * rs * gs / float(p.D);
#pragma unroll
    for (int k = 0; k < NU; ++k) {
      const int u = lane + 64 * k;
      if (u >= nu) continue;
      float ds[4];
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        ds[e] = rs * dy[k][e] * wv[k][e] - c * s[k][e];
        if (p.dro) ds[e] += dro[k][e];
        dwacc[k][e] = fmaf(dy[k][e] * s[k][e], rs, dwacc[k][e]);
      }
      store4(p.dx, int64_t(row) * p.dx_sr + 4 * u, p.dx_f32, ds);
      if (p.dres) store4(p.dres, int64_t(row) * p.dres_sr + 4 * u, p.dres_f32, ds);
    }
  }
#pragma unroll
  for (int k = 0; k < NU; ++k) {
    const int u = lane + 64 * k;
    if (u < nu)
#pragma unroll
      for (int e = 0; e < 4; ++e) red[wave][4 * u + e] = dwacc[k][e];
  }
  __syncthreads();
  for (int d = threadIdx.x; d < p.D; d += 64 * NW) {
    float a = 0.f;
#pragma unroll
    for (int w = 0; w < NW; ++w) a += red[w][d];
    p.part[int64_t(blockIdx.x) * p.D + d] = a;
  }
}

// dw = the fixed-order sum of the workgroups' partials. A workgroup owns 64 elements (one per lane, so
// a wave reads 256 contiguous bytes of a partial); wave w adds partials w, w + 16, ... (all of them in
// flight at once for up to 256 partials), then wave 0 adds the 16 wave sums in order.
__global__ void __launch_bounds__(64 * kNormDwWaves) add_rms_norm_dw_kernel(const float* part, int nparts, int D,
                                                                             float* dw) {
  __shared__ float red[kNormDwWaves][64];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int d = blockIdx.x * 64 + lane;
  const int dc = min(d, D - 1);
  float v[16];
#pragma unroll
  for (int j = 0; j < 16; ++j) {
    const int i = wave + j * kNormDwWaves;
    v[j] = i < nparts ? part[int64_t(i) * D + dc] : 0.f;
  }
  float a = 0.f;
#pragma unroll
  for (int j = 0; j < 16; ++j) a += v[j];
  for (int i = wave + 16 * kNormDwWaves; i < nparts; i += kNormDwWaves) a += part[int64_t(i) * D + dc];
  red[wave][lane] = a;
  __syncthreads();
  if (wave == 0 && d < D) {
    float t = 0.f;
#pragma unroll
    for (int w = 0; w < kNormDwWaves; ++w) t += red[w][lane];
    dw[d] = t;
  }
}

// ------------------------------------------------------------------------------------------------
// host side
// ------------------------------------------------------------------------------------------------
static int norm_units(int D) { return D <= 256 ? 1 : D <= 512 ? 2 : D <= 1024 ? 4 : 8; }

static bool al(const void* ptr, int64_t sr, bool f32) {
  const int64_t need = f32 ? 16 : 8;
  const int64_t es = f32 ? 4 : 2;
  return ptr == nullptr || ((reinterpret_cast<uintptr_t>(ptr) % need == 0) && (sr * es) % need == 0);
}

static int norm_check(int D, int rows) {
  if (D <= 0 || D % 4 != 0 || D > 2048)
    return set_error(MOTE_ERR_SHAPE, "add_rms_norm: D = %d unsupported (need 4 <= D <= 2048, D %% 4 == 0)", D);
  if (rows < 0) return set_error(MOTE_ERR_SHAPE, "add_rms_norm: rows = %d", rows);
  return MOTE_OK;
}

static int dt_ok(int dt) { return dt == MOTE_F32 || dt == MOTE_BF16; }

int launch_add_rms_norm_fwd(const mote_add_rms_norm_args* a, hipStream_t stream) {
  if (!a) return set_error(MOTE_ERR_ARGUMENT, "add_rms_norm_fwd: null args");
  int rc = norm_check(a->D, a->rows);
  if (rc) return rc;
  if (!dt_ok(a->dtype) || !dt_ok(a->out_dtype) || (a->residual && !dt_ok(a->res_dtype)) ||
      (a->residual_out && !dt_ok(a->res_out_dtype)))
    return set_error(MOTE_ERR_ARGUMENT, "add_rms_norm_fwd: bad dtype");
  if (a->rows == 0) return MOTE_OK;   // empty tensors may carry null data pointers
  if (!a->x || !a->weight || !a->y) return set_error(MOTE_ERR_ARGUMENT, "add_rms_norm_fwd: null pointer");
  NormParams p;
  p.x = a->x; p.x_sr = a->x_sr; p.res = a->residual; p.r_sr = a->res_sr; p.w = a->weight;
  p.y = a->y; p.y_sr = a->y_sr; p.res_out = a->residual_out; p.ro_sr = a->res_out_sr; p.rstd = a->rstd;
  p.rows = a->rows; p.D = a->D; p.eps = a->eps;
  p.x_f32 = a->dtype == MOTE_F32; p.res_f32 = a->res_dtype == MOTE_F32; p.out_f32 = a->out_dtype == MOTE_F32;
  p.res_out_f32 = a->res_out_dtype == MOTE_F32;
  p.round_sum = a->residual != nullptr && a->res_out_dtype == MOTE_BF16;
  if (!al(p.x, p.x_sr, p.x_f32) || !al(p.res, p.r_sr, p.res_f32) || !al(p.y, p.y_sr, p.out_f32) ||
      !al(p.res_out, p.ro_sr, p.res_out_f32) || reinterpret_cast<uintptr_t>(p.w) % 16)
    return set_error(MOTE_ERR_ARGUMENT, "add_rms_norm_fwd: rows must start on 8-byte (bf16) / 16-byte (fp32) boundaries");
  const int blocks = (a->rows + kNormWaves - 1) / kNormWaves;
  switch (norm_units(a->D)) {
    case 1: hipLaunchKernelGGL(add_rms_norm_fwd_kernel<1>, dim3(blocks), dim3(64 * kNormWaves), 0, stream, p); break;
    case 2: hipLaunchKernelGGL(add_rms_norm_fwd_kernel<2>, dim3(blocks), dim3(64 * kNormWaves), 0, stream, p); break;
    case 4: hipLaunchKernelGGL(add_rms_norm_fwd_kernel<4>, dim3(blocks), dim3(64 * kNormWaves), 0, stream, p); break;
    default: hipLaunchKernelGGL(add_rms_norm_fwd_kernel<8>, dim3(blocks), dim3(64 * kNormWaves), 0, stream, p); break;
  }
  return check_launch("add_rms_norm_fwd");
}

// waves per backward workgroup: 16 while a lane's registers allow (D <= 1024), else 8
static int norm_bwd_waves(int D) { return norm_units(D) <= 4 ? 16 : 8; }

// workgroups of the backward: one per CU at most, so that the dw partials stay few
static int norm_bwd_blocks(int rows, int D) {
  const int nw = norm_bwd_waves(D);
  const int want = (rows + nw - 1) / nw;
  return want < kNormBwdBlocks ? (want < 1 ? 1 : want) : kNormBwdBlocks;
}

size_t add_rms_norm_bwd_workspace_bytes(const mote_add_rms_norm_bwd_args* a) {
  return size_t(norm_bwd_blocks(a->rows, a->D)) * size_t(a->D > 0 ? a->D : 0) * sizeof(float);
}

int launch_add_rms_norm_bwd(const mote_add_rms_norm_bwd_args* a, hipStream_t stream) {
  if (!a) return set_error(MOTE_ERR_ARGUMENT, "add_rms_norm_bwd: null args");
  int rc = norm_check(a->D, a->rows);
  if (rc) return rc;
  if (!dt_ok(a->dtype) || !dt_ok(a->s_dtype) || (a->dres_out && !dt_ok(a->dres_out_dtype)) ||
      (a->dresidual && !dt_ok(a->dres_dtype)) || !dt_ok(a->dx_dtype))
    return set_error(MOTE_ERR_ARGUMENT, "add_rms_norm_bwd: bad dtype");
  if (!a->dweight) return set_error(MOTE_ERR_ARGUMENT, "add_rms_norm_bwd: null pointer");
  if (a->rows == 0) {                 // no rows: dw = 0 (a sum over no partials)
    hipLaunchKernelGGL(add_rms_norm_dw_kernel, dim3((a->D + 63) / 64), dim3(64 * kNormDwWaves), 0, stream,
                       static_cast<const float*>(nullptr), 0, a->D, a->dweight);
    return check_launch("add_rms_norm_bwd/dw");
  }
  if (!a->dy || !a->s || !a->rstd || !a->weight || !a->dx || !a->dweight)
    return set_error(MOTE_ERR_ARGUMENT, "add_rms_norm_bwd: null pointer");
  if (!a->workspace || a->workspace_bytes < add_rms_norm_bwd_workspace_bytes(a))
    return set_error(MOTE_ERR_WORKSPACE, "add_rms_norm_bwd: workspace too small");
  NormBwdParams p;
  p.dy = a->dy; p.dy_sr = a->dy_sr; p.dro = a->dres_out; p.dro_sr = a->dres_out_sr; p.s = a->s; p.s_sr = a->s_sr;
  p.rstd = a->rstd; p.w = a->weight; p.dx = a->dx; p.dx_sr = a->dx_sr; p.dres = a->dresidual;
  p.dres_sr = a->dres_sr; p.part = reinterpret_cast<float*>(a->workspace); p.dw = a->dweight;
  p.rows = a->rows; p.D = a->D;
  p.dy_f32 = a->dtype == MOTE_F32; p.dro_f32 = a->dres_out_dtype == MOTE_F32; p.s_f32 = a->s_dtype == MOTE_F32;
  p.dx_f32 = a->dx_dtype == MOTE_F32; p.dres_f32 = a->dres_dtype == MOTE_F32;
  if (!al(p.dy, p.dy_sr, p.dy_f32) || !al(p.dro, p.dro_sr, p.dro_f32) || !al(p.s, p.s_sr, p.s_f32) ||
      !al(p.dx, p.dx_sr, p.dx_f32) || !al(p.dres, p.dres_sr, p.dres_f32) || reinterpret_cast<uintptr_t>(p.w) % 16)
    return set_error(MOTE_ERR_ARGUMENT, "add_rms_norm_bwd: rows must start on 8-byte (bf16) / 16-byte (fp32) boundaries");
  const int blocks = norm_bwd_blocks(a->rows, a->D);
  const dim3 grid(blocks), b16(64 * 16), b8(64 * 8);
  switch (norm_units(a->D)) {
    case 1: hipLaunchKernelGGL((add_rms_norm_bwd_kernel<1, 16>), grid, b16, 0, stream, p); break;
    case 2: hipLaunchKernelGGL((add_rms_norm_bwd_kernel<2, 16>), grid, b16, 0, stream, p); break;
    case 4: hipLaunchKernelGGL((add_rms_norm_bwd_kernel<4, 16>), grid, b16, 0, stream, p); break;
    default: hipLaunchKernelGGL((add_rms_norm_bwd_kernel<8, 8>), grid, b8, 0, stream, p); break;
  }
  rc = check_launch("add_rms_norm_bwd");
  if (rc) return rc;
  hipLaunchKernelGGL(add_rms_norm_dw_kernel, dim3((a->D + 63) / 64), dim3(64 * kNormDwWaves), 0, stream, p.part,
                     blocks, a->D, a->dweight);
  return check_launch("add_rms_norm_bwd/dw");
}

}  // namespace mote
