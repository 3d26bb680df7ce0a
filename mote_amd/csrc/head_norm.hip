// Backward of QK-Norm (HeadRMSNorm, mote/model/relation.py:71-94, applied to p1 / p2 at :208-210)
// for the fused projection prologue: per head row of the raw projection x (before the norm) with
// g = dy * gain and r = (mean(x^2) + eps)^(-1/2):
//   dx = r g - r^3 x mean(g x),      dgain = sum over rows and heads of dy x r,
// in fp32 from bf16 inputs, dx rounded to bf16 (the eager autograd of the reference's fp32 norm).
//
// Four lanes per head row (D / 4 consecutive elements each, whole 16-byte chunks), so a row's two
// sums take two lane swaps; a workgroup of 256 threads covers 64 head rows at a time. The grid
// holds a multiple of (parts x H) head-row slots, so every slot keeps one (part, head) for the whole
// loop and its lanes accumulate dgain partials for fixed gain elements in registers. Each workgroup
// adds its slots' partials in a fixed order into one row of the workspace; a second launch adds the
// rows in order. Both orders are fixed, so dgain is bitwise reproducible.
#include "common.hpp"
#include "params.hpp"

namespace mote {

struct HeadNormBwdParams {
  const bf16_t* x;
  const bf16_t* dy;
  bf16_t* dx;
  int64_t x_sr, dy_sr, dx_sr;
  const float* gain0;
  const float* gain1;
  float* part;  // [gridDim.x][parts * D]
  int rows, parts, H;
  float eps;
};

constexpr int kHnSlots = 64;  // head rows per workgroup pass (4 lanes each)

template <int D>
__global__ void __launch_bounds__(256) head_norm_bwd_kernel(const HeadNormBwdParams p) {
  constexpr int E = D / 4, NC = E / 8;  // elements and 16-byte chunks per lane
  __shared__ float red[kHnSlots][4][E];
  const int tid = threadIdx.x, slot = tid >> 2, q = tid & 3;
  const int upr = p.parts * p.H;  // head rows per token row
  const int g0 = blockIdx.x * kHnSlots + slot;
  const int unit = g0 % upr, part = unit / p.H, head = unit - part * p.H;
  const int row_step = gridDim.x * kHnSlots / upr;
  const int64_t col = int64_t(part) * p.H * D + head * D + q * E;
  const float* gp = part ? p.gain1 : p.gain0;
  float gain[E], acc[E];
#pragma unroll
  for (int e = 0; e < E; ++e) {
    gain[e] = gp[q * E + e];
    acc[e] = 0.f;
  }
  constexpr float inv_d = 1.0f / D;
  for (int row = g0 / upr; row < p.rows; row += row_step) {
    uint4 xc[NC], dc[NC];
#pragma unroll
    for (int c = 0; c < NC; ++c) {
      xc[c] = *reinterpret_cast<const uint4*>(p.x + int64_t(row) * p.x_sr + col + 8 * c);
      dc[c] = *reinterpret_cast<const uint4*>(p.dy + int64_t(row) * p.dy_sr + col + 8 * c);
    }
    float xv[E], dv[E];
#pragma unroll
    for (int c = 0; c < NC; ++c) {
      const uint32_t xw[4] = {xc[c].x, xc[c].y, xc[c].z, xc[c].w};
      const uint32_t dw[4] = {dc[c].x, dc[c].y, dc[c].z, dc[c].w};
#pragma unroll
      for (int w = 0; w < 4; ++w) {
        xv[8 * c + 2 * w] = __uint_as_float(xw[w] << 16);
        xv[8 * c + 2 * w + 1] = __uint_as_float(xw[w] & 0xffff0000u);
        dv[8 * c + 2 * w] = __uint_as_float(dw[w] << 16);
        dv[8 * c + 2 * w + 1] = __uint_as_float(dw[w] & 0xffff0000u);
      }
    }
    float ss = 0.f, sgx = 0.f;
#pragma unroll
    for (int e = 0; e < E; ++e) {
      ss = fmaf(xv[e], xv[e], ss);
      sgx = fmaf(dv[e] * gain[e], xv[e], sgx);
    }
    // the row's four lanes are adjacent: two swaps give every lane the row's sums
    ss += __shfl_xor(ss, 1, 64);
    sgx += __shfl_xor(sgx, 1, 64);
    ss += __shfl_xor(ss, 2, 64);
    sgx += __shfl_xor(sgx, 2, 64);
    const float r = rsqrtf(ss * inv_d + p.eps);
    const float k3 = r * r * r * (sgx * inv_d);
    uint4 oc[NC];
#pragma unroll
    for (int c = 0; c < NC; ++c) {
      uint32_t ow[4];
#pragma unroll
      for (int w = 0; w < 4; ++w) {
        float o[2];
#pragma unroll
        for (int h = 0; h < 2; ++h) {
          const int e = 8 * c + 2 * w + h;
          o[h] = r * (dv[e] * gain[e]) - k3 * xv[e];
          acc[e] = fmaf(dv[e] * xv[e], r, acc[e]);
        }
        ow[w] = uint32_t(f2bf(o[0])) | (uint32_t(f2bf(o[1])) << 16);
      }
      oc[c] = uint4{ow[0], ow[1], ow[2], ow[3]};
    }
#pragma unroll
    for (int c = 0; c < NC; ++c) *reinterpret_cast<uint4*>(p.dx + int64_t(row) * p.dx_sr + col + 8 * c) = oc[c];
  }
#pragma unroll
  for (int e = 0; e < E; ++e) red[slot][q][e] = acc[e];
  __syncthreads();
  // the workgroup's partial of gain element j of part pj: its slots of that part, in slot order
  for (int j = tid; j < p.parts * D; j += 256) {
    const int pj = j / D, d = j - pj * D, qj = d / E, e = d - qj * E;
    float s = 0.f;
    for (int sl = 0; sl < kHnSlots; ++sl)
      if (((blockIdx.x * kHnSlots + sl) % upr) / p.H == pj) s += red[sl][qj][e];
    p.part[int64_t(blockIdx.x) * p.parts * D + j] = s;
  }
}

// dgain[j] = the workgroups' partials of element j added in workgroup order.
__global__ void __launch_bounds__(256) head_norm_sum_kernel(const float* part, int nblocks, int n, int D,
                                                            float* dgain0, float* dgain1) {
  const int j = threadIdx.x;
  if (j >= n) return;
  float s = 0.f;
  for (int b = 0; b < nblocks; ++b) s += part[int64_t(b) * n + j];
  if (j < D)
    dgain0[j] = s;
  else
    dgain1[j - D] = s;
}

static int gcd_int(int a, int b) {
  while (b) {
    const int t = a % b;
    a = b;
    b = t;
  }
  return a;
}

// Workgroups: enough 64-slot passes to give every head row a slot a few times over (at most 1024),
// rounded up to a multiple that makes the slot count a multiple of parts x H.
static int head_norm_blocks(const mote_head_norm_bwd_args* a) {
  const int upr = a->parts * a->H;
  const int m = upr / gcd_int(kHnSlots, upr);
  const int64_t units = int64_t(a->rows) * upr;
  int nb = int((units + kHnSlots * 4 - 1) / (kHnSlots * 4));
  nb = nb < 1 ? 1 : (nb > 1024 ? 1024 : nb);
  return (nb + m - 1) / m * m;
}

}  // namespace mote

extern "C" size_t mote_head_rms_norm_bwd_workspace(const mote_head_norm_bwd_args* a) {
  if (!a || a->parts < 1 || a->parts > 2 || a->H <= 0 || a->D <= 0) return 0;
  return size_t(mote::head_norm_blocks(a)) * a->parts * a->D * sizeof(float);
}

extern "C" int mote_head_rms_norm_bwd(const mote_head_norm_bwd_args* a, void* stream_) {
  using namespace mote;
  if (!a) return set_error(MOTE_ERR_ARGUMENT, "mote_head_rms_norm_bwd: null arguments");
  if (a->dtype != MOTE_BF16) return set_error(MOTE_ERR_ARGUMENT, "mote_head_rms_norm_bwd: bf16 tensors only");
  if (a->parts < 1 || a->parts > 2 || a->H <= 0 || a->rows < 0)
    return set_error(MOTE_ERR_ARGUMENT, "mote_head_rms_norm_bwd: parts must be 1 or 2, H > 0, rows >= 0");
  if (a->D != 32 && a->D != 64 && a->D != 96 && a->D != 128)
    return set_error(MOTE_ERR_SHAPE, "mote_head_rms_norm_bwd: head dim %d (supported: 32, 64, 96, 128)", a->D);
  if (!a->x || !a->dy || !a->dx || !a->gain0 || !a->dgain0 || (a->parts == 2 && (!a->gain1 || !a->dgain1)))
    return set_error(MOTE_ERR_ARGUMENT, "mote_head_rms_norm_bwd: null tensor pointer");
  const auto aligned = [](const void* ptr, int64_t sr) {
    return (reinterpret_cast<uintptr_t>(ptr) & 15) == 0 && sr % 8 == 0;
  };
  if (!aligned(a->x, a->x_sr) || !aligned(a->dy, a->dy_sr) || !aligned(a->dx, a->dx_sr))
    return set_error(MOTE_ERR_ARGUMENT, "mote_head_rms_norm_bwd: rows must be 16-byte aligned");
  const size_t need = mote_head_rms_norm_bwd_workspace(a);
  if (!a->workspace || a->workspace_bytes < need)
    return set_error(MOTE_ERR_WORKSPACE, "mote_head_rms_norm_bwd: workspace of %zu bytes, %zu needed",
                     a->workspace_bytes, need);
  hipStream_t stream = reinterpret_cast<hipStream_t>(stream_);
  HeadNormBwdParams p;
  p.x = static_cast<const bf16_t*>(a->x);
  p.dy = static_cast<const bf16_t*>(a->dy);
  p.dx = static_cast<bf16_t*>(a->dx);
  p.x_sr = a->x_sr;
  p.dy_sr = a->dy_sr;
  p.dx_sr = a->dx_sr;
  p.gain0 = a->gain0;
  p.gain1 = a->parts == 2 ? a->gain1 : a->gain0;
  p.part = static_cast<float*>(a->workspace);
  p.rows = a->rows;
  p.parts = a->parts;
  p.H = a->H;
  p.eps = a->eps;
  const int nb = head_norm_blocks(a);
  switch (a->D) {
    case 32: hipLaunchKernelGGL(head_norm_bwd_kernel<32>, dim3(nb), dim3(256), 0, stream, p); break;
    case 64: hipLaunchKernelGGL(head_norm_bwd_kernel<64>, dim3(nb), dim3(256), 0, stream, p); break;
    case 96: hipLaunchKernelGGL(head_norm_bwd_kernel<96>, dim3(nb), dim3(256), 0, stream, p); break;
    default: hipLaunchKernelGGL(head_norm_bwd_kernel<128>, dim3(nb), dim3(256), 0, stream, p); break;
  }
  hipLaunchKernelGGL(head_norm_sum_kernel, dim3(1), dim3(256), 0, stream, p.part, nb, a->parts * a->D, a->D,
                     a->dgain0, a->parts == 2 ? a->dgain1 : a->dgain0);
  return check_launch("mote_head_rms_norm_bwd");
}
