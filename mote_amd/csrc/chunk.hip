// Chunking on either side of the main network: the ChunkLayer gather (mote/model/dc.py:192-218), the
// DeChunkLayer EMA and its expansion back to bytes (dc.py:221-340), their backwards, and the decode
// step of the EMA (dc.py:342-352).
//
// Route. Per row, the inclusive boundary count cum[t] and the stable order the reference gets from
// argsort(t + L * !mask) (dc.py:212-214): boundary positions in order, then the others in order, so
// position t goes to dest(t) = cum[t] - 1 (boundary) or num + t - cum[t] (other). One workgroup per
// row: a block scan over 16 positions per thread, then the permutation written by destination.
//
// EMA (z_m = p_m x_m + (1 - p_m) z_{m-1} over the chunks of a row; p clamped to [eps, 1 - eps]).
// The chunk axis is cut into segments of 64 chunks; a wave owns 128 channels (2 per lane, fp32
// arithmetic) of one segment, a workgroup four consecutive segments. Phase 1 runs each segment from
// zero (its end value e_s and decay A_s = prod (1 - p)) and the workgroup composes its four in order
// through LDS into one aggregate. Phase 2 folds the earlier workgroups' aggregates into the carry in
// order, then the workgroup's earlier segments, runs the segment again from it, keeps
// w_m = x_m - z_{m-1} (fp32, for the backward) and writes z_m to every byte of chunk m, i.e. bytes
// [perm[m], perm[m + 1]) (the last chunk to L): out[t] = z[cum[t] - 1] as dc.py:329-335 gathers it.
// The segments and workgroups are fixed, so the arithmetic that produces z_m depends on chunks <= m
// only: the result is causal bit for bit, as the reference keeps its own (dc.py:265-268).
// The backward mirrors this with a reverse scan g_m = ds_m + (1 - p_{m+1}) g_{m+1}, ds_m the sum of
// the output gradient over chunk m's bytes (workgroup aggregates composed from the last segment down,
// folded from the row's end); dx_m = p_m g_m, dp_m = sum_d g_m (x_m - z_{m-1}) (a fixed-order sum over
// channel strips), scattered to boundary_prob[..., 1] through the clamp.
#include "common.hpp"
#include "params.hpp"

namespace mote {

// ------------------------------------------------------------------------------------------------
// route
// ------------------------------------------------------------------------------------------------
constexpr int kRouteThreads = 1024;
constexpr int kRoutePer = 16;

struct RouteParams {
  const uint8_t* mask; int64_t mask_sr;
  int32_t* cum; int32_t* perm; int32_t* num;
  int32_t* cu;                     // cu_seqlens, written here when there is one row (else null)
  int L, vec, vec4, vecp;          // vec: mask rows on 16-byte boundaries; vec4: cum rows too; vecp: perm rows
};

// exclusive prefix of v over the workgroup (in thread order) and the workgroup's total
__device__ __forceinline__ int block_excl_scan(int v, int* sh, int& total) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, nw = blockDim.x >> 6;
  int x = v;
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    const int y = __shfl_up(x, o, 64);
    if (lane >= o) x += y;
  }
  if (lane == 63) sh[wave] = x;
  __syncthreads();
  int pre = 0, tot = 0;
  for (int w = 0; w < nw; ++w) {
    const int s = sh[w];
    pre += w < wave ? s : 0;
    tot += s;
  }
  __syncthreads();
  total = tot;
  return pre + x - v;
}

__global__ void __launch_bounds__(kRouteThreads) chunk_route_kernel(const RouteParams p) {
  __shared__ int sh[kRouteThreads / 64];
  __shared__ __align__(16) int sperm[kRouteThreads * kRoutePer];  // one tile's permutation, by destination
  const int b = blockIdx.x;
  const uint8_t* mk = p.mask + int64_t(b) * p.mask_sr;
  int32_t* cum = p.cum + int64_t(b) * p.L;
  int32_t* perm = p.perm + int64_t(b) * p.L;
  constexpr int tile = kRouteThreads * kRoutePer;
  if (p.L <= tile) {
    // one tile: the thread's flags stay in registers, the permutation follows the scan directly
    const int s = threadIdx.x * kRoutePer;
    int f[kRoutePer], c = 0;
    if (p.vec && s + kRoutePer <= p.L) {
      const uint4 v = *reinterpret_cast<const uint4*>(mk + s);
      const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
      for (int k = 0; k < kRoutePer; ++k) f[k] = ((w[k >> 2] >> (8 * (k & 3))) & 0xffu) != 0;
    } else {
#pragma unroll
      for (int k = 0; k < kRoutePer; ++k) f[k] = (s + k < p.L) ? (mk[s + k] != 0) : 0;
    }
#pragma unroll
    for (int k = 0; k < kRoutePer; ++k) c += f[k];
    int n;
    int run = block_excl_scan(c, sh, n);
    int cv[kRoutePer];
#pragma unroll
    for (int k = 0; k < kRoutePer; ++k) {
      const int t = s + k;
      run += f[k];
      cv[k] = run;
      if (t < p.L) sperm[f[k] ? run - 1 : n + t - run] = t;  // scattered in LDS, not in memory
    }
    if (p.vec4 && s + kRoutePer <= p.L) {
#pragma unroll
      for (int k = 0; k < kRoutePer; k += 4)
        *reinterpret_cast<int4*>(cum + s + k) = make_int4(cv[k], cv[k + 1], cv[k + 2], cv[k + 3]);
    } else {
#pragma unroll
      for (int k = 0; k < kRoutePer; ++k)
        if (s + k < p.L) cum[s + k] = cv[k];
    }
    if (threadIdx.x == 0) {
      p.num[b] = n;
      if (p.cu) { p.cu[0] = 0; p.cu[1] = n; }   // one row: cu_seqlens here, no second launch
    }
    __syncthreads();
    // the permutation out in order: 16-byte stores of consecutive entries when the row allows
    if (p.vecp) {
      for (int i = threadIdx.x; i < p.L / 4; i += kRouteThreads)
        reinterpret_cast<int4*>(perm)[i] = reinterpret_cast<const int4*>(sperm)[i];
    } else {
      for (int i = threadIdx.x; i < p.L; i += kRouteThreads) perm[i] = sperm[i];
    }
    return;
  }
  // longer rows: pass 1 writes cum tile by tile, pass 2 reads back the entries the thread wrote
  int carry = 0;
  for (int t0 = 0; t0 < p.L; t0 += tile) {
    const int s = t0 + threadIdx.x * kRoutePer;
    int f[kRoutePer], c = 0;
#pragma unroll
    for (int k = 0; k < kRoutePer; ++k) {
      f[k] = (s + k < p.L) ? (mk[s + k] != 0) : 0;
      c += f[k];
    }
    int total;
    int run = carry + block_excl_scan(c, sh, total);
#pragma unroll
    for (int k = 0; k < kRoutePer; ++k) {
      run += f[k];
      if (s + k < p.L) cum[s + k] = run;
    }
    carry += total;
  }
  const int n = carry;
  if (threadIdx.x == 0) p.num[b] = n;
  for (int t0 = 0; t0 < p.L; t0 += tile) {
    const int s = t0 + threadIdx.x * kRoutePer;
#pragma unroll
    for (int k = 0; k < kRoutePer; ++k) {
      const int t = s + k;
      if (t < p.L) {
        const int c = cum[t];
        const int dest = mk[t] ? c - 1 : n + t - c;
        perm[dest] = t;
      }
    }
  }
}

// cu_seqlens[b + 1] = num[0] + ... + num[b] (one workgroup, rows in order)
__global__ void __launch_bounds__(kRouteThreads) chunk_cu_kernel(const int32_t* num, int B, int32_t* cu) {
  __shared__ int sh[kRouteThreads / 64];
  int carry = 0;
  if (threadIdx.x == 0) cu[0] = 0;
  for (int b0 = 0; b0 < B; b0 += kRouteThreads) {
    const int b = b0 + threadIdx.x;
    const int v = b < B ? num[b] : 0;
    int total;
    const int pre = carry + block_excl_scan(v, sh, total);
    if (b < B) cu[b + 1] = pre + v;
    carry += total;
  }
}

// ------------------------------------------------------------------------------------------------
// gather (forward) and its backward: whole rows in 16-byte units, one wave per row
// ------------------------------------------------------------------------------------------------
struct GatherParams {
  const uint8_t* src; int64_t s_sb, s_sr;  // bytes
  uint8_t* dst; int64_t d_sb, d_sr;        // bytes
  const int32_t* perm; const int32_t* num; const int32_t* cu;
  const uint8_t* mask; int64_t mask_sr; const int32_t* cum;
  int B, L, M, row_units;                  // row_units: 16-byte units per row
};

__device__ __forceinline__ void copy_row(const uint8_t* s, uint8_t* d, int units, int lane) {
  for (int u = lane; u < units; u += 64)
    reinterpret_cast<uint4*>(d)[u] = reinterpret_cast<const uint4*>(s)[u];
}
__device__ __forceinline__ void zero_row(uint8_t* d, int units, int lane) {
  for (int u = lane; u < units; u += 64) reinterpret_cast<uint4*>(d)[u] = make_uint4(0, 0, 0, 0);
}

// out row (b, m) = hidden row (b, perm[b, m]); packed (cu != null): rows m < num[b] to row cu[b] + m
__global__ void __launch_bounds__(256) chunk_gather_kernel(const GatherParams p) {
  const int lane = threadIdx.x & 63;
  const int64_t r = int64_t(blockIdx.x) * 4 + (threadIdx.x >> 6);
  if (r >= int64_t(p.B) * p.M) return;
  const int b = int(r / p.M), m = int(r % p.M);
  const int t = p.perm[int64_t(b) * p.L + m];
  const uint8_t* s = p.src + b * p.s_sb + t * p.s_sr;
  if (p.cu) {
    if (m >= p.num[b]) return;
    copy_row(s, p.dst + int64_t(p.cu[b] + m) * p.d_sr, p.row_units, lane);
  } else {
    copy_row(s, p.dst + b * p.d_sb + m * p.d_sr, p.row_units, lane);
  }
}

// d hidden row (b, t) = d out row dest(t) when it was gathered, else zero
__global__ void __launch_bounds__(256) chunk_gather_bwd_kernel(const GatherParams p) {
  const int lane = threadIdx.x & 63;
  const int64_t r = int64_t(blockIdx.x) * 4 + (threadIdx.x >> 6);
  if (r >= int64_t(p.B) * p.L) return;
  const int b = int(r / p.L), t = int(r % p.L);
  const int c = p.cum[int64_t(b) * p.L + t];
  const bool bd = p.mask[b * p.mask_sr + t] != 0;
  uint8_t* d = p.dst + b * p.d_sb + t * p.d_sr;  // d hidden [B, L, D]
  if (p.cu) {
    if (bd) copy_row(p.src + int64_t(p.cu[b] + c - 1) * p.s_sr, d, p.row_units, lane);
    else zero_row(d, p.row_units, lane);
    return;
  }
  const int dest = bd ? c - 1 : p.num[b] + t - c;
  if (dest < p.M) copy_row(p.src + b * p.s_sb + dest * p.s_sr, d, p.row_units, lane);
  else zero_row(d, p.row_units, lane);
}

// ------------------------------------------------------------------------------------------------
// EMA dechunk
// ------------------------------------------------------------------------------------------------
constexpr int kDcCh = 128;        // channels per wave (2 per lane)
constexpr int kDcSeg = 64;        // chunks per segment (one lane per chunk for the per-chunk values)
constexpr int kDcGrp = 4;         // segments (waves) per workgroup: their carries combine through LDS, so
                                  // only the workgroups' aggregates cross workgroups

struct DechunkParams {
  const void* x; int64_t x_sb, x_sr;        // hidden [B, M, D] (elements)
  const void* prob; int64_t p_sb, p_sr;     // boundary_prob [B, L, 2] (elements; p at +1)
  const int32_t* perm; const int32_t* num;
  const int32_t* cum;                       // [B, L] inclusive boundary count (single-pass kernels)
  const float* init;                        // [B, D] carried value, or null
  void* out; int64_t o_sb, o_sr;            // [B, L, D] (forward)
  float* w;                                 // [B, M, D] fp32: x_m - z_{m-1}, kept for the backward (may be null)
  const void* dout; int64_t g_sb, g_sr;     // [B, L, D] (backward)
  void* dx; int64_t dx_sb, dx_sr;           // [B, M, D] (backward)
  float* ds;                                // [B, M, D] fp32: dout summed over each chunk's bytes (backward)
  float* segv; float* segd;                 // [B, nseg, D] segment values, [B, nseg] decays (backward)
  float* grpv; float* grpd;                 // [B, ngrp, D] workgroup aggregates' values, [B, ngrp] decays
  float* pc;                                // [B, M] clamped p of every chunk (vector path, kept by phase 1;
                                            // the backward's is negative where the clamp was active)
  void* dprob; int64_t dp_sb, dp_sr; int dp_f32;  // d boundary_prob [B, L, 2] (backward, vector path)
  float* part;                              // [B, nstrips, M] dp partials (backward)
  int B, L, M, D, nseg, ngrp, nstrips, p_f32;
  float eps;
};

// two consecutive elements as stored: float2 (fp32) or one 32-bit word (bf16 pair)
template <bool F32> struct Pair;
template <> struct Pair<true> {
  typedef float2 T;
  static __device__ __forceinline__ T ld(const void* base, int64_t off) {
    return *reinterpret_cast<const float2*>(reinterpret_cast<const float*>(base) + off);
  }
  static __device__ __forceinline__ float2 cvt(T v) { return v; }
  static __device__ __forceinline__ void st(void* base, int64_t off, float2 v) {
    *reinterpret_cast<float2*>(reinterpret_cast<float*>(base) + off) = v;
  }
};
template <> struct Pair<false> {
  typedef uint32_t T;
  static __device__ __forceinline__ T ld(const void* base, int64_t off) {
    return *reinterpret_cast<const uint32_t*>(reinterpret_cast<const bf16_t*>(base) + off);
  }
  static __device__ __forceinline__ float2 cvt(T v) { return make_float2(bf2f(v & 0xffffu), bf2f(v >> 16)); }
  static __device__ __forceinline__ void st(void* base, int64_t off, float2 v) {
    *reinterpret_cast<uint32_t*>(reinterpret_cast<bf16_t*>(base) + off) =
        uint32_t(f2bf(v.x)) | (uint32_t(f2bf(v.y)) << 16);
  }
};

__device__ __forceinline__ float ld1(const void* base, int64_t off, bool f32) {
  return f32 ? reinterpret_cast<const float*>(base)[off] : bf2f(reinterpret_cast<const bf16_t*>(base)[off]);
}
__device__ __forceinline__ float rdl(float v, int i) {
  return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), i));
}
__device__ __forceinline__ int rdl(int v, int i) { return __builtin_amdgcn_readlane(v, i); }

__device__ __forceinline__ float2 ldf2(const float* base, int64_t off) {
  return *reinterpret_cast<const float2*>(base + off);
}
__device__ __forceinline__ void stf2(float* base, int64_t off, float2 v) {
  *reinterpret_cast<float2*>(base + off) = v;
}

// chunks of row b that carry values: all of num (at most M); without a carried value a row with no
// boundary still has chunk 0 (every byte reads it, dc.py:327)
__device__ __forceinline__ int dc_used(const DechunkParams& p, int b) {
  const int n = min(p.num[b], p.M);
  return (p.init == nullptr && n == 0 && p.M > 0) ? 1 : n;
}

// p of chunk m (clamped), m < n
__device__ __forceinline__ float dc_p(const DechunkParams& p, int b, int m) {
  const int t = p.perm[int64_t(b) * p.L + m];
  const float v = ld1(p.prob, b * p.p_sb + int64_t(t) * p.p_sr + 1, p.p_f32);
  return fminf(fmaxf(v, p.eps), 1.0f - p.eps);
}

// first byte of chunk m (chunk 0 starts at byte 0 without a carried value), L past the last chunk
__device__ __forceinline__ int dc_lo(const DechunkParams& p, int b, int m, int n) {
  if (m >= n) return p.L;
  if (m == 0 && p.init == nullptr) return 0;
  return p.perm[int64_t(b) * p.L + m];
}

// c <- A_j c + e_j over the aggregates j = j0, j0 + step, ... (cnt of them) at gv (value rows of D
// floats) / gd (decays), in batches of 16, the next batch loading while the current one folds
__device__ __forceinline__ void dc_fold(const float* gv, const float* gd, int D, int d, int j0, int step, int cnt,
                                        float2& c) {
  float2 ea[16], eb[16];
  float Aa[16], Ab[16];
  auto load = [&](float2 (&e)[16], float (&A)[16], int k0) {
#pragma unroll
    for (int k = 0; k < 16; ++k) {
      const int j = j0 + step * min(k0 + k, cnt - 1);
      e[k] = ldf2(gv, int64_t(j) * D + d);
      A[k] = gd[j];
    }
  };
  auto fold = [&](float2 (&e)[16], float (&A)[16], int k0) {
#pragma unroll
    for (int k = 0; k < 16; ++k) {
      if (k0 + k < cnt) {
        c.x = fmaf(A[k], c.x, e[k].x);
        c.y = fmaf(A[k], c.y, e[k].y);
      }
    }
  };
  if (cnt <= 0) return;
  load(ea, Aa, 0);
  for (int k0 = 0; k0 < cnt; k0 += 32) {
    load(eb, Ab, k0 + 16);
    fold(ea, Aa, k0);
    if (k0 + 16 >= cnt) break;
    load(ea, Aa, k0 + 32);
    fold(eb, Ab, k0 + 16);
  }
}

// A wave's segment of the forward EMA: its chunks, their p (lane i holds chunk m0 + i) and x rows
// (loaded up front, clamped, unconditional), run from zero to its end value e and decay A.
template <bool F32>
struct DcFwdSeg {
  typedef Pair<F32> P;
  int m0, cnt;
  float pv;
  typename P::T xr[kDcSeg];
  float2 e;
  float A;
  __device__ __forceinline__ void run(const DechunkParams& p, int b, int d, int s, int n) {
    m0 = min(s * kDcSeg, n);
    cnt = min(kDcSeg, n - m0);
    e = make_float2(0.f, 0.f);
    A = 1.f;
    pv = 0.f;
    if (cnt <= 0) return;
    pv = dc_p(p, b, m0 + min(threadIdx.x & 63, cnt - 1));
    const int64_t xb = b * p.x_sb + d;
#pragma unroll
    for (int i = 0; i < kDcSeg; ++i) xr[i] = P::ld(p.x, xb + int64_t(m0 + min(i, cnt - 1)) * p.x_sr);
#pragma unroll
    for (int i = 0; i < kDcSeg; ++i) {
      const float pc = i < cnt ? rdl(pv, i) : 0.f;  // past the segment: p = 0 leaves e and A as they are
      const float a = 1.f - pc;
      const float2 x = P::cvt(xr[i]);
      e.x = fmaf(a, e.x, pc * x.x);
      e.y = fmaf(a, e.y, pc * x.y);
      A *= a;
    }
  }
};

// phase 1 (forward): every wave runs its segment from zero; the workgroup composes its kDcGrp
// segments in order (through LDS) into one aggregate (value, decay) for the later workgroups
template <bool F32>
__global__ void __launch_bounds__(64 * kDcGrp) dechunk_grp_kernel(const DechunkParams p) {
  __shared__ float2 se[kDcGrp][64];
  __shared__ float sa[kDcGrp];
  const int lane = threadIdx.x & 63, w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int strip = blockIdx.x, g = blockIdx.y, b = blockIdx.z;
  const int d = min(strip * kDcCh + 2 * lane, p.D - 2);
  DcFwdSeg<F32> sg;
  sg.run(p, b, d, g * kDcGrp + w, dc_used(p, b));
  se[w][lane] = sg.e;
  if (lane == 0) sa[w] = sg.A;
  __syncthreads();
  if (w == 0) {
    float2 e = make_float2(0.f, 0.f);
    float A = 1.f;
#pragma unroll
    for (int i = 0; i < kDcGrp; ++i) {
      const float a = sa[i];
      e.x = fmaf(a, e.x, se[i][lane].x);
      e.y = fmaf(a, e.y, se[i][lane].y);
      A *= a;
    }
    const int64_t gi = int64_t(b) * p.ngrp + g;
    if (strip * kDcCh + 2 * lane < p.D) stf2(p.grpv, gi * p.D + d, e);
    if (strip == 0 && lane == 0) p.grpd[gi] = A;
  }
}

// phase 2 (forward): the carry into the workgroup (the row's carried value, then the earlier
// workgroups' aggregates in order), into the wave (its workgroup's earlier segments, from LDS), then
// the segment again from it: w_m = x_m - z_{m-1} (fp32, for the backward) and z_m written to every
// byte of chunk m (bytes [first byte of m, first byte of m + 1); dc.py:329-335 gathers the same
// values by the boundary count); bytes before the first boundary hold the carried value with one.
template <bool F32>
__global__ void __launch_bounds__(64 * kDcGrp) dechunk_out_kernel(const DechunkParams p) {
  typedef Pair<F32> P;
  __shared__ float2 se[kDcGrp][64];
  __shared__ float sa[kDcGrp];
  const int lane = threadIdx.x & 63, w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int strip = blockIdx.x, g = blockIdx.y, b = blockIdx.z;
  const int s = g * kDcGrp + w;
  const bool live = strip * kDcCh + 2 * lane < p.D;
  const int d = min(strip * kDcCh + 2 * lane, p.D - 2);
  const int n = dc_used(p, b);
  DcFwdSeg<F32> sg;
  sg.run(p, b, d, s, n);
  // the lane's chunk's byte range (lanes past the segment: empty)
  const int t0l = sg.cnt > 0 ? dc_lo(p, b, sg.m0 + lane, n) : p.L;
  const int t1l = sg.cnt > 0 ? dc_lo(p, b, sg.m0 + lane + 1, n) : p.L;
  se[w][lane] = sg.e;
  if (lane == 0) sa[w] = sg.A;
  float2 c = make_float2(0.f, 0.f);
  if (p.init) c = ldf2(p.init, int64_t(b) * p.D + d);
  dc_fold(p.grpv + int64_t(b) * p.ngrp * p.D, p.grpd + int64_t(b) * p.ngrp, p.D, d, 0, 1, g, c);
  __syncthreads();
  for (int i = 0; i < w; ++i) {
    const float a = sa[i];
    c.x = fmaf(a, c.x, se[i][lane].x);
    c.y = fmaf(a, c.y, se[i][lane].y);
  }
  const int64_t ob = b * p.o_sb + d;
  if (s == 0 && p.init) {
    const int tf = dc_lo(p, b, 0, n);
    for (int t = 0; t < tf; ++t)
      if (live) P::st(p.out, ob + int64_t(t) * p.o_sr, c);
  }
  if (sg.cnt <= 0) return;
  float2 z = c;
  float* wrow = p.w + (int64_t(b) * p.M + sg.m0) * p.D + d;
#pragma unroll
  for (int i = 0; i < kDcSeg; ++i) {
    if (i < sg.cnt) {
      const float pc = rdl(sg.pv, i), a = 1.f - pc;
      const float2 x = P::cvt(sg.xr[i]);
      if (live && p.w) stf2(wrow, int64_t(i) * p.D, make_float2(x.x - z.x, x.y - z.y));
      z.x = fmaf(a, z.x, pc * x.x);
      z.y = fmaf(a, z.y, pc * x.y);
      const int t0 = rdl(t0l, i), t1 = rdl(t1l, i);
      for (int t = t0; t < t1; ++t)
        if (live) P::st(p.out, ob + int64_t(t) * p.o_sr, z);
    }
  }
}

// backward: ds[b, m] = dout summed over chunk m's bytes, in byte order (fp32); one wave per chunk row,
// 8 channels per lane (16-byte loads when rows allow), 4 byte rows in flight
template <bool F32>
__global__ void __launch_bounds__(256) dechunk_dsum_kernel(const DechunkParams p, int vec) {
  const int lane = threadIdx.x & 63;
  const int64_t r = int64_t(blockIdx.x) * 4 + (threadIdx.x >> 6);
  if (r >= int64_t(p.B) * p.M) return;
  const int b = int(r / p.M), m = int(r % p.M);
  // the count and both positions in one round trip (m < M <= L); dc_used / dc_lo from them
  const int nraw = p.num[b];
  const int pa = p.perm[int64_t(b) * p.L + m];
  const int pb = p.perm[int64_t(b) * p.L + min(m + 1, p.L - 1)];
  const int n0 = min(nraw, p.M);
  const int n = (p.init == nullptr && n0 == 0 && p.M > 0) ? 1 : n0;
  if (m >= n) return;
  const int t0 = (m == 0 && p.init == nullptr) ? 0 : pa;
  const int t1 = m + 1 >= n ? p.L : pb;
  float* dsrow = p.ds + (int64_t(b) * p.M + m) * p.D;
  const int64_t gb = b * p.g_sb;
  for (int d0 = 8 * lane; d0 < p.D; d0 += 512) {
    float acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
    if (vec) {  // D % 8 == 0, rows on 16-byte boundaries
      for (int t = t0; t < t1; t += 4) {
        float v[4][8];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const int64_t off = gb + int64_t(min(t + j, t1 - 1)) * p.g_sr + d0;
          if (F32) {
            const float4 a0 = *reinterpret_cast<const float4*>(reinterpret_cast<const float*>(p.dout) + off);
            const float4 a1 = *reinterpret_cast<const float4*>(reinterpret_cast<const float*>(p.dout) + off + 4);
            v[j][0] = a0.x; v[j][1] = a0.y; v[j][2] = a0.z; v[j][3] = a0.w;
            v[j][4] = a1.x; v[j][5] = a1.y; v[j][6] = a1.z; v[j][7] = a1.w;
          } else {
            const uint4 a = *reinterpret_cast<const uint4*>(reinterpret_cast<const bf16_t*>(p.dout) + off);
            const uint32_t w[4] = {a.x, a.y, a.z, a.w};
#pragma unroll
            for (int k = 0; k < 4; ++k) {
              v[j][2 * k] = bf2f(w[k] & 0xffffu);
              v[j][2 * k + 1] = bf2f(w[k] >> 16);
            }
          }
        }
#pragma unroll
        for (int j = 0; j < 4; ++j)
          if (t + j < t1)
#pragma unroll
            for (int k = 0; k < 8; ++k) acc[k] += v[j][k];
      }
      *reinterpret_cast<float4*>(dsrow + d0) = make_float4(acc[0], acc[1], acc[2], acc[3]);
      *reinterpret_cast<float4*>(dsrow + d0 + 4) = make_float4(acc[4], acc[5], acc[6], acc[7]);
    } else {
      const int nv = min(8, p.D - d0);  // even
      for (int t = t0; t < t1; ++t) {
        const int64_t off = gb + int64_t(t) * p.g_sr + d0;
        for (int k = 0; k < nv; k += 2) {
          float2 v;
          if (F32) {
            v = *reinterpret_cast<const float2*>(reinterpret_cast<const float*>(p.dout) + off + k);
          } else {
            const uint32_t w = *reinterpret_cast<const uint32_t*>(reinterpret_cast<const bf16_t*>(p.dout) + off + k);
            v = make_float2(bf2f(w & 0xffffu), bf2f(w >> 16));
          }
          acc[k] += v.x;
          acc[k + 1] += v.y;
        }
      }
      for (int k = 0; k < nv; k += 2) stf2(dsrow, d0 + k, make_float2(acc[k], acc[k + 1]));
    }
  }
}

// phase 1 (backward): every wave runs the reverse scan of its segment from zero over its ds rows
// (loaded up front): h_m = ds_m + (1 - p_{m+1}) h_{m+1}; it keeps the value at the first chunk and the
// decay prod_{k = m0+1}^{m0+cnt} (1 - p_k) that carries the next segment's value into it (segments
// past the row: value 0, decay 1). The workgroup composes its segments from the last down (LDS)
// into one aggregate for the earlier workgroups.
__global__ void __launch_bounds__(64 * kDcGrp) dechunk_bwd_grp_kernel(const DechunkParams p) {
  __shared__ float2 sh[kDcGrp][64];
  __shared__ float sa[kDcGrp];
  const int lane = threadIdx.x & 63, w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int strip = blockIdx.x, g = blockIdx.y, b = blockIdx.z;
  const int s = g * kDcGrp + w;
  const bool live = strip * kDcCh + 2 * lane < p.D;
  const int d = min(strip * kDcCh + 2 * lane, p.D - 2);
  const int n = dc_used(p, b);
  const int m0 = min(s * kDcSeg, n), cnt = min(kDcSeg, n - m0);
  float2 h = make_float2(0.f, 0.f);
  float A = 1.f;
  if (cnt > 0) {
    const int mm = m0 + min(lane, cnt - 1);
    const float pn = mm + 1 < n ? dc_p(p, b, mm + 1) : 0.f;  // p of the next chunk
    float2 dsr[kDcSeg];
    const int64_t db = (int64_t(b) * p.M + m0) * p.D + d;
#pragma unroll
    for (int i = 0; i < kDcSeg; ++i) dsr[i] = ldf2(p.ds, db + int64_t(min(i, cnt - 1)) * p.D);
#pragma unroll
    for (int i = kDcSeg - 1; i >= 0; --i) {
      if (i < cnt) {
        const float an = 1.f - rdl(pn, i);
        h.x = fmaf(an, h.x, dsr[i].x);
        h.y = fmaf(an, h.y, dsr[i].y);
        A *= an;
      }
    }
  }
  const int64_t si = int64_t(b) * p.nseg + s;
  if (live) stf2(p.segv, si * p.D + d, h);
  if (strip == 0 && lane == 0) p.segd[si] = A;
  sh[w][lane] = h;
  if (lane == 0) sa[w] = A;
  __syncthreads();
  if (w == 0) {
    float2 e = make_float2(0.f, 0.f);
    float Ag = 1.f;
#pragma unroll
    for (int i = kDcGrp - 1; i >= 0; --i) {
      const float a = sa[i];
      e.x = fmaf(a, e.x, sh[i][lane].x);
      e.y = fmaf(a, e.y, sh[i][lane].y);
      Ag *= a;
    }
    const int64_t gi = int64_t(b) * p.ngrp + g;
    if (live) stf2(p.grpv, gi * p.D + d, e);
    if (strip == 0 && lane == 0) p.grpd[gi] = Ag;
  }
}

// phase 2 (backward): the carry into the segment's end from the later workgroups' aggregates (from
// the row's last down) and the later segments of its own workgroup, then the reverse run again over
// ds: dx = p g and the dp partials sum_d g (x - z_prev) = sum_d g w, reduced over the wave's channels
// in a fixed order. ds and w rows come in 4 stages of 16 chunks, the next stage loading while the
// current one runs.
template <bool F32>
__global__ void __launch_bounds__(64 * kDcGrp) dechunk_bwd_out_kernel(const DechunkParams p) {
  typedef Pair<F32> P;
  __shared__ float red[kDcGrp][kDcSeg][65];
  const int lane = threadIdx.x & 63, w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int strip = blockIdx.x, g = blockIdx.y, b = blockIdx.z;
  const int s = g * kDcGrp + w;
  const bool live = strip * kDcCh + 2 * lane < p.D;
  const int d = min(strip * kDcCh + 2 * lane, p.D - 2);
  const int n = dc_used(p, b);
  const int m0 = min(s * kDcSeg, n), cnt = min(kDcSeg, n - m0);
  const int64_t xb = b * p.dx_sb + d;
  if (s == p.nseg - 1) {  // rows no byte reads: zero gradient
    for (int m = n; m < p.M; ++m)
      if (live) P::st(p.dx, xb + int64_t(m) * p.dx_sr, make_float2(0.f, 0.f));
  }
  if (cnt > 0) {
    const int mm = m0 + min(lane, cnt - 1);
    const float pv = dc_p(p, b, mm);
    const float pn = mm + 1 < n ? dc_p(p, b, mm + 1) : 0.f;
    const int64_t db = (int64_t(b) * p.M + m0) * p.D + d;
    float2 dsa[16], wa[16], dsb[16], wb[16];
    auto load = [&](float2 (&dsv)[16], float2 (&wv)[16], int q) {
#pragma unroll
      for (int k = 0; k < 16; ++k) {
        const int i = min(16 * q + k, cnt - 1);
        dsv[k] = ldf2(p.ds, db + int64_t(i) * p.D);
        wv[k] = ldf2(p.w, db + int64_t(i) * p.D);
      }
    };
    load(dsa, wa, 3);
    // G = g at chunk m0 + cnt: the row's later workgroups (last .. g + 1), then the workgroup's later
    // segments (kDcGrp - 1 .. w + 1), each G <- f + A' G
    float2 gg = make_float2(0.f, 0.f);
    const int lastg = ((n + kDcSeg - 1) / kDcSeg - 1) / kDcGrp;
    dc_fold(p.grpv + int64_t(b) * p.ngrp * p.D, p.grpd + int64_t(b) * p.ngrp, p.D, d, lastg, -1, lastg - g, gg);
    for (int i = kDcGrp - 1; i > w; --i) {
      const int64_t sj = int64_t(b) * p.nseg + g * kDcGrp + i;
      const float a = p.segd[sj];
      const float2 f = ldf2(p.segv, sj * p.D + d);
      gg.x = fmaf(a, gg.x, f.x);
      gg.y = fmaf(a, gg.y, f.y);
    }
    auto run = [&](float2 (&dsv)[16], float2 (&wv)[16], int q) {
#pragma unroll
      for (int k = 15; k >= 0; --k) {
        const int i = 16 * q + k;
        if (i < cnt) {
          const float an = 1.f - rdl(pn, i), pc = rdl(pv, i);
          gg.x = fmaf(an, gg.x, dsv[k].x);
          gg.y = fmaf(an, gg.y, dsv[k].y);
          if (live) P::st(p.dx, xb + int64_t(m0 + i) * p.dx_sr, make_float2(pc * gg.x, pc * gg.y));
          red[w][i][lane] = live ? gg.x * wv[k].x + gg.y * wv[k].y : 0.f;
        }
      }
    };
    load(dsb, wb, 2);
    run(dsa, wa, 3);
    load(dsa, wa, 1);
    run(dsb, wb, 2);
    load(dsb, wb, 0);
    run(dsa, wa, 1);
    run(dsb, wb, 0);
  }
  __syncthreads();
  if (lane < cnt) {  // lane k sums chunk m0 + k over the 64 lanes, in lane order
    float a = 0.f;
    for (int l = 0; l < 64; ++l) a += red[w][lane][l];
    p.part[(int64_t(b) * p.nstrips + strip) * p.M + m0 + lane] = a;
  }
}

// ------------------------------------------------------------------------------------------------
// Eight consecutive elements of a row (vector path: D % 8 == 0, rows on 16-byte boundaries) as one
// 16-byte (bf16) or two 16-byte (fp32) accesses. Every launch of the vector path is a chain of
// dependent memory round trips, so each issues every load that needs no other at its start (rows
// clamped to the bucket M before the row's chunk count arrives, which then only masks).
// ------------------------------------------------------------------------------------------------
template <bool F32> struct V8;
template <> struct V8<false> {  // 8 bf16
  struct Raw { uint4 u; };
  static __device__ __forceinline__ Raw ld(const void* base, int64_t off) {
    return Raw{*reinterpret_cast<const uint4*>(reinterpret_cast<const bf16_t*>(base) + off)};
  }
  static __device__ __forceinline__ void cvt(const Raw& r, float (&v)[8]) {
    const uint32_t w[4] = {r.u.x, r.u.y, r.u.z, r.u.w};
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      v[2 * k] = bf2f(w[k] & 0xffffu);
      v[2 * k + 1] = bf2f(w[k] >> 16);
    }
  }
  static __device__ __forceinline__ void st(void* base, int64_t off, const float (&v)[8]) {
    uint32_t w[4];
#pragma unroll
    for (int k = 0; k < 4; ++k) w[k] = uint32_t(f2bf(v[2 * k])) | (uint32_t(f2bf(v[2 * k + 1])) << 16);
    *reinterpret_cast<uint4*>(reinterpret_cast<bf16_t*>(base) + off) = uint4{w[0], w[1], w[2], w[3]};
  }
  static __device__ __forceinline__ Raw pack(const float (&v)[8]) {
    uint32_t w[4];
#pragma unroll
    for (int k = 0; k < 4; ++k) w[k] = uint32_t(f2bf(v[2 * k])) | (uint32_t(f2bf(v[2 * k + 1])) << 16);
    return Raw{uint4{w[0], w[1], w[2], w[3]}};
  }
  static __device__ __forceinline__ void st_raw(void* base, int64_t off, const Raw& r) {
    *reinterpret_cast<uint4*>(reinterpret_cast<bf16_t*>(base) + off) = r.u;
  }
};
template <> struct V8<true> {  // 8 fp32
  struct Raw { float4 a, b; };
  static __device__ __forceinline__ Raw ld(const void* base, int64_t off) {
    const float4* q = reinterpret_cast<const float4*>(reinterpret_cast<const float*>(base) + off);
    return Raw{q[0], q[1]};
  }
  static __device__ __forceinline__ void cvt(const Raw& r, float (&v)[8]) {
    v[0] = r.a.x; v[1] = r.a.y; v[2] = r.a.z; v[3] = r.a.w; v[4] = r.b.x; v[5] = r.b.y; v[6] = r.b.z; v[7] = r.b.w;
  }
  static __device__ __forceinline__ void st(void* base, int64_t off, const float (&v)[8]) {
    float4* q = reinterpret_cast<float4*>(reinterpret_cast<float*>(base) + off);
    q[0] = make_float4(v[0], v[1], v[2], v[3]);
    q[1] = make_float4(v[4], v[5], v[6], v[7]);
  }
  static __device__ __forceinline__ Raw pack(const float (&v)[8]) {
    return Raw{make_float4(v[0], v[1], v[2], v[3]), make_float4(v[4], v[5], v[6], v[7])};
  }
  static __device__ __forceinline__ void st_raw(void* base, int64_t off, const Raw& r) {
    float4* q = reinterpret_cast<float4*>(reinterpret_cast<float*>(base) + off);
    q[0] = r.a;
    q[1] = r.b;
  }
};
typedef V8<true> F8;

// the row's chunk count (dc_used) from the raw count
__device__ __forceinline__ int dc_used_raw(const DechunkParams& p, int nraw) {
  const int n = min(nraw, p.M);
  return (p.init == nullptr && n == 0 && p.M > 0) ? 1 : n;
}
__device__ __forceinline__ float dc_clamp(const DechunkParams& p, float v) {
  return fminf(fmaxf(v, p.eps), 1.0f - p.eps);
}

// d boundary_prob: [..., 0] = 0, [..., 1] = dp of the chunk the position starts (fixed-order sum over
// the channel strips), passed through the clamp
__global__ void __launch_bounds__(256) dechunk_dprob_kernel(const DechunkParams p, const uint8_t* mask,
                                                            int64_t mask_sr, const int32_t* cum, void* dprob,
                                                            int64_t dp_sb, int64_t dp_sr, int dp_f32) {
  const int64_t r = int64_t(blockIdx.x) * 256 + threadIdx.x;
  if (r >= int64_t(p.B) * p.L) return;
  const int b = int(r / p.L), t = int(r % p.L);
  const int n = dc_used(p, b);
  int m = -1;
  if (mask[b * mask_sr + t]) m = cum[int64_t(b) * p.L + t] - 1;
  else if (t == 0 && p.num[b] == 0 && n == 1) m = 0;  // the row's only chunk is byte 0
  float v = 0.f;
  if (m >= 0 && m < n) {
    for (int k = 0; k < p.nstrips; ++k) v += p.part[(int64_t(b) * p.nstrips + k) * p.M + m];
    const float raw = ld1(p.prob, b * p.p_sb + int64_t(t) * p.p_sr + 1, p.p_f32);
    if (!(raw >= p.eps && raw <= 1.0f - p.eps)) v = 0.f;
  }
  const int64_t off = b * dp_sb + int64_t(t) * dp_sr;
  if (dp_f32) {
    reinterpret_cast<float*>(dprob)[off] = 0.f;
    reinterpret_cast<float*>(dprob)[off + 1] = v;
  } else {
    reinterpret_cast<bf16_t*>(dprob)[off] = 0;
    reinterpret_cast<bf16_t*>(dprob)[off + 1] = f2bf(v);
  }
}

// Backward chunk sums, balanced by bytes (vector path): one wave per kDsBytes bytes of a row sums the
// chunks that start in them, each over all of its bytes (past the range when the last one continues),
// in byte order from zero, 8 channels per lane over the row in slabs of 512: the sums of
// dechunk_dsum_kernel bit for bit. A wave's work is its range plus one chunk, wherever the boundaries
// fall, and the chunk changes are the same for every lane (no divergence).
constexpr int kDsBytes = 16;

template <bool F32>
__global__ void __launch_bounds__(64) dechunk_dsum_bal_kernel(const DechunkParams p) {
  typedef V8<F32> V;
  const int lane = threadIdx.x & 63;
  const int R0 = blockIdx.x * kDsBytes, b = blockIdx.y;
  if (R0 >= p.L) return;
  const int32_t* cum = p.cum + int64_t(b) * p.L;
  const int32_t* perm = p.perm + int64_t(b) * p.L;
  const int n = dc_used_raw(p, p.num[b]);
  // chunks ka .. kb - 1 start in [R0, R0 + kDsBytes): chunk 0 at byte 0, chunk k >= 1 at perm[k]
  const int ka = min(R0 == 0 ? 0 : max(cum[R0 - 1], 1), n);
  const int kb = min(max(cum[min(R0 + kDsBytes, p.L) - 1], R0 == 0 ? 1 : 0), n);
  if (ka >= kb) return;
  // lane i: the first byte past chunk ka + i (its end), for the chunks of the range (at most kDsBytes)
  const int ke = ka + lane;
  const int endl = ke + 1 >= n ? p.L : perm[min(ke + 1, p.L - 1)];
  const int t_lo = ka == 0 ? 0 : perm[ka];
  const int t_hi = __builtin_amdgcn_readlane(endl, kb - 1 - ka);
  const int64_t gb = b * p.g_sb;
  for (int d0 = 0; d0 < p.D; d0 += 512) {
    const int d = min(d0 + 8 * lane, p.D - 8);
    const bool live = d0 + 8 * lane < p.D;
    float acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
    int k = ka, kend = __builtin_amdgcn_readlane(endl, 0);
    constexpr int NR = F32 ? 8 : 16;
    typename V::Raw ra[NR], rb[NR];
    auto load = [&](typename V::Raw (&rr)[NR], int t0) {
#pragma unroll
      for (int j = 0; j < NR; ++j) rr[j] = V::ld(p.dout, gb + int64_t(min(t0 + j, t_hi - 1)) * p.g_sr + d);
    };
    auto add = [&](const typename V::Raw (&rr)[NR], int t0) {
#pragma unroll
      for (int j = 0; j < NR; ++j) {
        const int t = t0 + j;
        if (t < t_hi) {  // uniform
          float v[8];
          V::cvt(rr[j], v);
#pragma unroll
          for (int c = 0; c < 8; ++c) acc[c] += v[c];
          if (t + 1 == kend) {  // chunk k ends here: its row of sums
            if (live) F8::st(p.ds + (int64_t(b) * p.M + k) * p.D, d, acc);
#pragma unroll
            for (int c = 0; c < 8; ++c) acc[c] = 0.f;
            ++k;
            kend = __builtin_amdgcn_readlane(endl, min(k - ka, 63));
          }
        }
      }
    };
    load(ra, t_lo);
    for (int t0 = t_lo; t0 < t_hi; t0 += 2 * NR) {
      if (t0 + NR < t_hi) load(rb, t0 + NR);
      add(ra, t0);
      if (t0 + 2 * NR < t_hi) load(ra, t0 + 2 * NR);
      if (t0 + NR < t_hi) add(rb, t0 + NR);
    }
  }
}

// ------------------------------------------------------------------------------------------------
// Vector path over 64-channel strips (D % 8 == 0, rows on 16-byte boundaries). A wave owns one
// 64-chunk segment of a 64-channel strip as eight 8-lane groups: group g runs chunks m0 + 8 g .. + 7
// and lane r of it channels 8 r .. 8 r + 7 (16-byte accesses), so a wave's sequential chain is 8
// chunks long and a row of 16 384 bytes keeps 640 waves busy at D = 512. Segments compose in groups
// of four. Two launches per direction: the first writes the segment and group aggregates to the
// workspace, the second reads them with plain loads. (A single-launch form whose waves exchanged the
// aggregates through coherent memory, with per-call epochs and bounded polling, measured no faster:
// two exchange hops of one to two round trips each cost more than the kernel boundary.)
// ------------------------------------------------------------------------------------------------
constexpr int kFsCh = 64;                // channels per strip
constexpr int kFsSub = 8;                // chunks per lane group (8 groups of 8 lanes)
constexpr int kFsMaxStrips = 8;          // backward: one wave per strip in a workgroup, D <= 512

// lane 8 g + i's value for the lanes of group g (i a constant): lane reads and a select, no LDS trip
template <typename T>
__device__ __forceinline__ T grp8(T v, int i, int g) {
  T a[8];
#pragma unroll
  for (int k = 0; k < 8; ++k) a[k] = rdl(v, 8 * k + i);
  T o = a[7];
#pragma unroll
  for (int k = 6; k >= 0; --k) o = g == k ? a[k] : o;
  return o;
}

// the maps (values E, decay A) held by the eight lane groups, composed in order g = 0 .. 7 (forward)
// or 7 .. 0 (backward) into c, their decays into Ac (every lane holds the result)
template <bool Rev>
__device__ __forceinline__ void grp_compose(const float (&E)[8], float A, int r, float (&c)[8], float& Ac) {
#pragma unroll
  for (int k = 0; k < 8; ++k) {
    const int gg = Rev ? 7 - k : k;
    const int src = 8 * gg + r;
    const float Ag = __shfl(A, src, 64);
#pragma unroll
    for (int ch = 0; ch < 8; ++ch) c[ch] = fmaf(Ag, c[ch], __shfl(E[ch], src, 64));
    Ac *= Ag;
  }
}

// c <- A_j c + e_j over workspace aggregates j = j0 + step k (k < cnt) in order: each 8-lane group
// composes an eighth (8 maps loaded at a time), then every lane applies the eighths in order
__device__ __forceinline__ void dw_fold(const float* gv, const float* gd, int D, int d, int j0, int step, int cnt,
                                        int r, int gq, float (&c)[8]) {
  const int per = (max(cnt, 0) + 7) / 8;
  const int k0 = gq * per, k1 = min(cnt, k0 + per);
  float E[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
  float A = 1.f;
  for (int kb = k0; kb < k1; kb += 8) {
    F8::Raw e[8];
    float a[8];
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      const int j = j0 + step * min(kb + k, k1 - 1);
      e[k] = F8::ld(gv, int64_t(j) * D + d);
      a[k] = gd[j];
    }
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      if (kb + k < k1) {
        float v[8];
        F8::cvt(e[k], v);
#pragma unroll
        for (int ch = 0; ch < 8; ++ch) E[ch] = fmaf(a[k], E[ch], v[ch]);
        A *= a[k];
      }
    }
  }
  float Ac = 1.f;
  grp_compose<false>(E, A, r, c, Ac);
}

// The same fold in two steps, for a kernel with registers to spare: issue() loads the first 8 maps of
// the group's eighth (all of them while cnt <= 64, i.e. M <= 16 384 chunks) at the kernel's start;
// fold() composes them with any remaining ones.
struct DwFold {
  const float* gv;
  const float* gd;
  int D, d, j0, step, k0, k1;
  F8::Raw e[8];
  float a[8];
  __device__ __forceinline__ void issue(const float* gv_, const float* gd_, int D_, int d_, int j0_, int step_,
                                        int cnt, int gq) {
    gv = gv_, gd = gd_, D = D_, d = d_, j0 = j0_, step = step_;
    const int per = (max(cnt, 0) + 7) / 8;
    k0 = gq * per;
    k1 = min(cnt, k0 + per);
    load(k0);
  }
  __device__ __forceinline__ void load(int kb) {
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      const int j = j0 + step * max(min(kb + k, k1 - 1), 0);
      e[k] = F8::ld(gv, int64_t(j) * D + d);
      a[k] = gd[j];
    }
  }
  __device__ __forceinline__ void fold(int r, float (&c)[8]) {
    float E[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
    float A = 1.f;
    for (int kb = k0; kb < k1; kb += 8) {
      if (kb > k0) load(kb);
#pragma unroll
      for (int k = 0; k < 8; ++k) {
        if (kb + k < k1) {
          float v[8];
          F8::cvt(e[k], v);
#pragma unroll
          for (int ch = 0; ch < 8; ++ch) E[ch] = fmaf(a[k], E[ch], v[ch]);
          A *= a[k];
        }
      }
    }
    float Ac = 1.f;
    grp_compose<false>(E, A, r, c, Ac);
  }
};

// phase 1 (forward): a workgroup per (strip, group of four segments, row), a wave per segment: the
// 8-chunk runs from zero, the segment's map (its lane groups in order) to segv / segd, the group's map
// (its segments in order, through LDS) to grpv / grpd, and the clamped p of every chunk to pc
template <bool F32>
__global__ void __launch_bounds__(64 * kDcGrp) dechunk_grp_w_kernel(const DechunkParams p) {
  typedef V8<F32> V;
  __shared__ float se[kDcGrp][8][8];
  __shared__ float sa[kDcGrp];
  const int lane = threadIdx.x & 63, w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int gq = lane >> 3, r = lane & 7;
  const int strip = blockIdx.x, g = blockIdx.y, b = blockIdx.z;
  const bool live = strip * kFsCh + 8 * r < p.D;
  const int d = min(strip * kFsCh + 8 * r, p.D - 8);
  const int s = g * kDcGrp + w, ms = s * kDcSeg, mq = ms + kFsSub * gq, mmax = max(p.M - 1, 0);
  const int nraw = p.num[b];
  const int tp = p.perm[int64_t(b) * p.L + min(ms + lane, mmax)];
  typename V::Raw xr[kFsSub];
  if (p.M > 0) {
#pragma unroll
    for (int i = 0; i < kFsSub; ++i) xr[i] = V::ld(p.x, b * p.x_sb + d + int64_t(min(mq + i, mmax)) * p.x_sr);
  }
  const float pv = dc_clamp(p, ld1(p.prob, b * p.p_sb + int64_t(tp) * p.p_sr + 1, p.p_f32));
  const int n = dc_used_raw(p, nraw);
  const int cnt = min(kDcSeg, n - ms), cs = min(max(cnt - kFsSub * gq, 0), kFsSub);
  if (strip == 0 && ms + lane < p.M) p.pc[int64_t(b) * p.M + ms + lane] = pv;
  float pcs[kFsSub];
#pragma unroll
  for (int i = 0; i < kFsSub; ++i) pcs[i] = grp8(pv, i, gq);
  float e[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
  float A = 1.f;
  if (cnt > 0) {
#pragma unroll
    for (int i = 0; i < kFsSub; ++i) {
      if (i < cs) {
        float x[8];
        V::cvt(xr[i], x);
        const float a = 1.f - pcs[i];
#pragma unroll
        for (int c = 0; c < 8; ++c) e[c] = fmaf(a, e[c], pcs[i] * x[c]);
        A *= a;
      }
    }
  }
  float S[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
  float As = 1.f;
  grp_compose<false>(e, A, r, S, As);
  const int64_t si = int64_t(b) * p.nseg + s;
  if (gq == 0) {
    if (live) F8::st(p.segv, si * p.D + d, S);
#pragma unroll
    for (int c = 0; c < 8; ++c) se[w][r][c] = S[c];
    if (r == 0) {
      sa[w] = As;
      if (strip == 0) p.segd[si] = As;
    }
  }
  __syncthreads();
  if (w == 0 && gq == 0) {
    float G[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
    float Ga = 1.f;
#pragma unroll
    for (int k = 0; k < kDcGrp; ++k) {
#pragma unroll
      for (int c = 0; c < 8; ++c) G[c] = fmaf(sa[k], G[c], se[k][r][c]);
      Ga *= sa[k];
    }
    const int64_t gi = int64_t(b) * p.ngrp + g;
    if (live) F8::st(p.grpv, gi * p.D + d, G);
    if (strip == 0 && r == 0) p.grpd[gi] = Ga;
  }
}

// phase 2 (forward): one wave per (strip, segment, row): the carry (the row's carried value, the
// earlier groups, the earlier segments of the group), the 8-chunk runs again with w and z (z to LDS in
// out's dtype), then the segment's bytes [T0, T1): byte t takes the z row of chunk cum[t] - 1, eight
// bytes per store instruction (group g takes byte T0 + 8 k + g, every store a whole 128-byte row
// piece), each block's LDS reads issued before its stores; the chunk indices of the first 256 bytes
// load at the kernel's start
template <bool F32>
__global__ void __launch_bounds__(64) dechunk_out_w_kernel(const DechunkParams p) {
  typedef V8<F32> V;
  __shared__ typename V::Raw zl[kDcSeg + 1][8];
  const int lane = threadIdx.x & 63, gq = lane >> 3, r = lane & 7;
  const int strip = blockIdx.x, s = blockIdx.y, b = blockIdx.z;
  const int g = s / kDcGrp, nsib = s - g * kDcGrp;
  const bool live = strip * kFsCh + 8 * r < p.D;
  const int d = min(strip * kFsCh + 8 * r, p.D - 8);
  const int ms = s * kDcSeg, mq = ms + kFsSub * gq, mmax = max(p.M - 1, 0);
  // every load that needs no other first
  const int nraw = p.num[b];
  const float pv = p.M > 0 ? p.pc[int64_t(b) * p.M + min(ms + lane, mmax)] : 0.f;
  const int pa = p.perm[int64_t(b) * p.L + min(ms + lane, mmax)];
  const int pb = p.perm[int64_t(b) * p.L + min(ms + lane + 1, mmax)];
  typename V::Raw xr[kFsSub];
  if (p.M > 0) {
#pragma unroll
    for (int i = 0; i < kFsSub; ++i) xr[i] = V::ld(p.x, b * p.x_sb + d + int64_t(min(mq + i, mmax)) * p.x_sr);
  }
  float z[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
  if (p.init) F8::cvt(F8::ld(p.init, int64_t(b) * p.D + d), z);
  F8::Raw sv[kDcGrp - 1];
  float sd[kDcGrp - 1];
#pragma unroll
  for (int k = 0; k < kDcGrp - 1; ++k) {
    const int64_t si = int64_t(b) * p.nseg + min(g * kDcGrp + k, s);
    sv[k] = F8::ld(p.segv, si * p.D + d);
    sd[k] = p.segd[si];
  }
  const int n = dc_used_raw(p, nraw);
  const int cnt = min(kDcSeg, n - ms), cs = min(max(cnt - kFsSub * gq, 0), kFsSub);
  const int pa0 = __shfl(pa, 0, 64), pb63 = __shfl(pb, 63, 64);
  const int T0 = s == 0 ? 0 : (ms < n ? pa0 : p.L);
  const int T1 = ms + kDcSeg < n ? pb63 : p.L;
  const int32_t* cum = p.cum + int64_t(b) * p.L;
  constexpr int kPre = 4;
  int cv[kPre * 8];
#pragma unroll
  for (int i = 0; i < kPre * 8; ++i) cv[i] = cum[max(min(T0 + 8 * i + gq, T1 - 1), 0)];
  DwFold gf;
  gf.issue(p.grpv + int64_t(b) * p.ngrp * p.D, p.grpd + int64_t(b) * p.ngrp, p.D, d, 0, 1, g, gq);
  // the lane group's chunks from zero (for the carry into each group), while the aggregates arrive
  float pcs[kFsSub];
#pragma unroll
  for (int i = 0; i < kFsSub; ++i) pcs[i] = grp8(pv, i, gq);
  float e[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
  float A = 1.f;
  if (cnt > 0) {
#pragma unroll
    for (int i = 0; i < kFsSub; ++i) {
      if (i < cs) {
        float x[8];
        V::cvt(xr[i], x);
        const float a = 1.f - pcs[i];
#pragma unroll
        for (int c = 0; c < 8; ++c) e[c] = fmaf(a, e[c], pcs[i] * x[c]);
        A *= a;
      }
    }
  }
  // the carry into the segment: the earlier groups, then the earlier segments of the group
  gf.fold(r, z);
#pragma unroll
  for (int k = 0; k < kDcGrp - 1; ++k) {
    if (k < nsib) {
      float v[8];
      F8::cvt(sv[k], v);
#pragma unroll
      for (int c = 0; c < 8; ++c) z[c] = fmaf(sd[k], z[c], v[c]);
    }
  }
  if (s == 0 && gq == 0) zl[kDcSeg][r] = V::pack(z);  // bytes before the first boundary (carried value)
#pragma unroll
  for (int gg = 0; gg < 7; ++gg) {
    const int src = 8 * gg + r;
    const float Ag = __shfl(A, src, 64);
    float Eg[8];
#pragma unroll
    for (int c = 0; c < 8; ++c) Eg[c] = __shfl(e[c], src, 64);
    if (gg < gq) {
#pragma unroll
      for (int c = 0; c < 8; ++c) z[c] = fmaf(Ag, z[c], Eg[c]);
    }
  }
  if (cnt > 0) {
    float* wrow = p.w ? p.w + (int64_t(b) * p.M + mq) * p.D + d : nullptr;
#pragma unroll
    for (int i = 0; i < kFsSub; ++i) {
      if (i < cs) {
        float x[8];
        V::cvt(xr[i], x);
        if (live && p.w) {
          float wv[8];
#pragma unroll
          for (int c = 0; c < 8; ++c) wv[c] = x[c] - z[c];
          F8::st(wrow, int64_t(i) * p.D, wv);
        }
        const float a = 1.f - pcs[i];
#pragma unroll
        for (int c = 0; c < 8; ++c) z[c] = fmaf(a, z[c], pcs[i] * x[c]);
        zl[kFsSub * gq + i][r] = V::pack(z);
      }
    }
  }
  __builtin_amdgcn_wave_barrier();  // one wave: LDS in order, no workgroup barrier
  const int64_t ob = b * p.o_sb + d;
  auto block = [&](int t0, const int* cb) {
    typename V::Raw zr[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      int c = cb[i] - 1;
      if (!p.init) c = max(c, 0);
      c = min(c, n - 1);
      zr[i] = zl[c < ms ? kDcSeg : min(c - ms, kDcSeg - 1)][r];
    }
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int t = t0 + 8 * i + gq;
      if (live && t < T1) V::st_raw(p.out, ob + int64_t(t) * p.o_sr, zr[i]);
    }
  };
#pragma unroll
  for (int k = 0; k < kPre; ++k)
    if (T0 + 64 * k < T1) block(T0 + 64 * k, cv + 8 * k);
  for (int t0 = T0 + 64 * kPre; t0 < T1; t0 += 64) {
    int cn[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) cn[i] = cum[min(t0 + 8 * i + gq, T1 - 1)];
    block(t0, cn);
  }
}

// phase 1 (backward): a workgroup per (strip, group of four segments, row), a wave per segment: the
// 8-chunk reverse runs from zero over the chunk sums, the segment's map (lane groups from the last) to
// segv / segd, the group's map (segments from the last, through LDS) to grpv / grpd, and the clamped
// p of every chunk to pc with the clamp's gradient gate in its sign (negative where it was clamped)
__global__ void __launch_bounds__(64 * kDcGrp) dechunk_bwd_grp_w_kernel(const DechunkParams p) {
  __shared__ float se[kDcGrp][8][8];
  __shared__ float sa[kDcGrp];
  const int lane = threadIdx.x & 63, w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int gq = lane >> 3, r = lane & 7;
  const int strip = blockIdx.x, g = blockIdx.y, b = blockIdx.z;
  const bool live = strip * kFsCh + 8 * r < p.D;
  const int d = min(strip * kFsCh + 8 * r, p.D - 8);
  const int s = g * kDcGrp + w, ms = s * kDcSeg, mq = ms + kFsSub * gq, mmax = p.M - 1;  // M >= 1 here
  const int nraw = p.num[b];
  const int ta = p.perm[int64_t(b) * p.L + min(ms + lane, mmax)];
  const int tb = p.perm[int64_t(b) * p.L + min(ms + lane + 1, mmax)];
  F8::Raw dsr[kFsSub];
#pragma unroll
  for (int i = 0; i < kFsSub; ++i) dsr[i] = F8::ld(p.ds, int64_t(b) * p.M * p.D + d + int64_t(min(mq + i, mmax)) * p.D);
  const float praw = ld1(p.prob, b * p.p_sb + int64_t(ta) * p.p_sr + 1, p.p_f32);
  const float pv = dc_clamp(p, praw);
  const float pnr = dc_clamp(p, ld1(p.prob, b * p.p_sb + int64_t(tb) * p.p_sr + 1, p.p_f32));
  const int n = dc_used_raw(p, nraw);
  const int cnt = min(kDcSeg, n - ms), cs = min(max(cnt - kFsSub * gq, 0), kFsSub);
  if (strip == 0 && ms + lane < p.M)
    p.pc[int64_t(b) * p.M + ms + lane] = (praw >= p.eps && praw <= 1.0f - p.eps) ? pv : -pv;
  const float pn = ms + lane + 1 < n ? pnr : 0.f;
  float h[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
  float A = 1.f;
  if (cnt > 0) {
#pragma unroll
    for (int i = kFsSub - 1; i >= 0; --i) {
      const float an = 1.f - grp8(pn, i, gq);
      if (i < cs) {
        float v[8];
        F8::cvt(dsr[i], v);
#pragma unroll
        for (int c = 0; c < 8; ++c) h[c] = fmaf(an, h[c], v[c]);
        A *= an;
      }
    }
  }
  float S[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
  float As = 1.f;
  grp_compose<true>(h, A, r, S, As);
  const int64_t si = int64_t(b) * p.nseg + s;
  if (gq == 0) {
    if (live) F8::st(p.segv, si * p.D + d, S);
#pragma unroll
    for (int c = 0; c < 8; ++c) se[w][r][c] = S[c];
    if (r == 0) {
      sa[w] = As;
      if (strip == 0) p.segd[si] = As;
    }
  }
  __syncthreads();
  if (w == 0 && gq == 0) {
    float G[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
    float Ga = 1.f;
#pragma unroll
    for (int k = kDcGrp - 1; k >= 0; --k) {
#pragma unroll
      for (int c = 0; c < 8; ++c) G[c] = fmaf(sa[k], G[c], se[k][r][c]);
      Ga *= sa[k];
    }
    const int64_t gi = int64_t(b) * p.ngrp + g;
    if (live) F8::st(p.grpv, gi * p.D + d, G);
    if (strip == 0 && r == 0) p.grpd[gi] = Ga;
  }
}

// phase 2 (backward): a workgroup per (segment, row), a wave per strip: the carry into the segment's
// end (the later groups from the last down, then the later siblings), the lane groups' later chunks,
// dx = p g, the dp partials (transposed butterfly over each group's 8 lanes), the strips' partials
// added in order through LDS and d boundary_prob over the segment's bytes
template <bool F32>
__global__ void __launch_bounds__(64 * kFsMaxStrips) dechunk_bwd_out_w_kernel(const DechunkParams p) {
  typedef V8<F32> V;
  __shared__ float red[kFsMaxStrips][kDcSeg];
  const int lane = threadIdx.x & 63, strip = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int gq = lane >> 3, r = lane & 7;
  const int s = blockIdx.x, b = blockIdx.y;
  const int g = s / kDcGrp, nsib = g * kDcGrp + kDcGrp - 1 - s;
  const bool live = strip * kFsCh + 8 * r < p.D;
  const int d = min(strip * kFsCh + 8 * r, p.D - 8);
  const int ms = s * kDcSeg, mq = ms + kFsSub * gq, mmax = p.M - 1;  // M >= 1 here
  const int nraw = p.num[b];
  const float pc_lane = p.pc[int64_t(b) * p.M + min(ms + lane, mmax)];
  const float pnr = fabsf(p.pc[int64_t(b) * p.M + min(ms + lane + 1, mmax)]);
  const int pa = p.perm[int64_t(b) * p.L + min(ms + lane, mmax)];
  const int pb = p.perm[int64_t(b) * p.L + min(ms + lane + 1, mmax)];
  F8::Raw dsr[kFsSub], wr[kFsSub];
#pragma unroll
  for (int i = 0; i < kFsSub; ++i) {
    const int64_t off = int64_t(b) * p.M * p.D + d + int64_t(min(mq + i, mmax)) * p.D;
    dsr[i] = F8::ld(p.ds, off);
    wr[i] = F8::ld(p.w, off);
  }
  F8::Raw sv[kDcGrp - 1];
  float sd[kDcGrp - 1];
#pragma unroll
  for (int k = 0; k < kDcGrp - 1; ++k) {
    const int64_t si = int64_t(b) * p.nseg + max(g * kDcGrp + kDcGrp - 1 - k, s);
    sv[k] = F8::ld(p.segv, si * p.D + d);
    sd[k] = p.segd[si];
  }
  const int n = dc_used_raw(p, nraw);
  const int cnt = min(kDcSeg, n - ms), cs = min(max(cnt - kFsSub * gq, 0), kFsSub);
  const float pn = ms + lane + 1 < n ? pnr : 0.f;
  const float pv = fabsf(pc_lane);
  float G[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
  dw_fold(p.grpv + int64_t(b) * p.ngrp * p.D, p.grpd + int64_t(b) * p.ngrp, p.D, d, p.ngrp - 1, -1,
          p.ngrp - 1 - g, r, gq, G);
#pragma unroll
  for (int k = 0; k < kDcGrp - 1; ++k) {
    if (k < nsib) {
      float v[8];
      F8::cvt(sv[k], v);
#pragma unroll
      for (int c = 0; c < 8; ++c) G[c] = fmaf(sd[k], G[c], v[c]);
    }
  }
  const int64_t xb = b * p.dx_sb + d;
  if (s == p.nseg - 1) {  // rows no byte reads: zero gradient, the groups taking turns
    const float zero[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
    for (int mz = n + gq; mz < p.M; mz += 8)
      if (live) V::st(p.dx, xb + int64_t(mz) * p.dx_sr, zero);
  }
  float mine = 0.f;
  if (cnt > 0) {
    float ans[kFsSub], pcs[kFsSub];
#pragma unroll
    for (int i = 0; i < kFsSub; ++i) {
      ans[i] = 1.f - grp8(pn, i, gq);
      pcs[i] = grp8(pv, i, gq);
    }
    // the lane group's chunks from zero, for the carry into each group from the later ones
    float h[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
    float A = 1.f;
#pragma unroll
    for (int i = kFsSub - 1; i >= 0; --i) {
      if (i < cs) {
        float v[8];
        F8::cvt(dsr[i], v);
#pragma unroll
        for (int c = 0; c < 8; ++c) h[c] = fmaf(ans[i], h[c], v[c]);
        A *= ans[i];
      }
    }
#pragma unroll
    for (int gg = 7; gg >= 1; --gg) {
      const int src = 8 * gg + r;
      const float Ag = __shfl(A, src, 64);
      float Hg[8];
#pragma unroll
      for (int c = 0; c < 8; ++c) Hg[c] = __shfl(h[c], src, 64);
      if (gg > gq) {
#pragma unroll
        for (int c = 0; c < 8; ++c) G[c] = fmaf(Ag, G[c], Hg[c]);
      }
    }
    float dots[kFsSub];
#pragma unroll
    for (int i = kFsSub - 1; i >= 0; --i) {
      dots[i] = 0.f;
      if (i < cs) {
        float v[8], wv[8], dx[8];
        F8::cvt(dsr[i], v);
        F8::cvt(wr[i], wv);
#pragma unroll
        for (int c = 0; c < 8; ++c) {
          G[c] = fmaf(ans[i], G[c], v[c]);
          dx[c] = pcs[i] * G[c];
        }
        if (live) {
          V::st(p.dx, xb + int64_t(mq + i) * p.dx_sr, dx);
          float dt = 0.f;
#pragma unroll
          for (int c = 0; c < 8; ++c) dt = fmaf(G[c], wv[c], dt);
          dots[i] = dt;
        }
      }
    }
    float t4[4], t2[2];
    const bool b2 = r & 4, b1 = r & 2, b0 = r & 1;
#pragma unroll
    for (int j = 0; j < 4; ++j) t4[j] = (b2 ? dots[j + 4] : dots[j]) + __shfl_xor(b2 ? dots[j] : dots[j + 4], 4, 64);
#pragma unroll
    for (int j = 0; j < 2; ++j) t2[j] = (b1 ? t4[j + 2] : t4[j]) + __shfl_xor(b1 ? t4[j] : t4[j + 2], 2, 64);
    mine = (b0 ? t2[1] : t2[0]) + __shfl_xor(b0 ? t2[0] : t2[1], 1, 64);
  }
  red[strip][lane] = mine;
  __syncthreads();
  if (strip == 0 && lane < cnt) {
    // chunk ms + lane: dp in strip order, gated by the clamp; its bytes [t0, t1) of d prob
    float dp = 0.f;
    for (int k = 0; k < p.nstrips; ++k) dp += red[k][lane];
    if (pc_lane < 0.f) dp = 0.f;
    const int t0 = ms + lane == 0 ? 0 : pa;  // no carried value in the backward
    const int t1 = ms + lane + 1 >= n ? p.L : pb;
    const int tb = nraw > 0 ? pa : 0;        // the boundary byte (byte 0 of a row without one)
    for (int t = t0; t < t1; ++t) {
      const float v = t == tb ? dp : 0.f;
      const int64_t off = b * p.dp_sb + int64_t(t) * p.dp_sr;
      if (p.dp_f32) {
        reinterpret_cast<float*>(p.dprob)[off] = 0.f;
        reinterpret_cast<float*>(p.dprob)[off + 1] = v;
      } else {
        reinterpret_cast<bf16_t*>(p.dprob)[off] = 0;
        reinterpret_cast<bf16_t*>(p.dprob)[off + 1] = f2bf(v);
      }
    }
  }
}

// ------------------------------------------------------------------------------------------------
// decode step: last <- p cur + (1 - p) last, every operation rounded to the state's dtype
// ------------------------------------------------------------------------------------------------
struct DcStepParams {
  const uint8_t* mask; const void* prob; int64_t p_sr; const void* hidden; int64_t h_sr;
  void* last; int64_t l_sr; void* out; int64_t o_sr;
  int B, D, p_f32, h_f32, s_f32;
  float eps;
};

__device__ __forceinline__ float rnd(float v, bool f32) { return f32 ? v : bf2f(f2bf(v)); }

__global__ void __launch_bounds__(256) dechunk_step_kernel(const DcStepParams p) {
  const int b = blockIdx.y;
  const int d = blockIdx.x * 256 + threadIdx.x;
  if (d >= p.D) return;
  const bool on = p.mask[b] != 0;
  int rank = 0;  // rows of hidden hold the boundary rows in batch order
  for (int j = 0; j < b; ++j) rank += p.mask[j] != 0;
  const bool sf = p.s_f32;
  float pb = 0.f, cur = 0.f;
  if (on) {
    const float raw = ld1(p.prob, int64_t(b) * p.p_sr + 1, p.p_f32);
    pb = rnd(rnd(fminf(fmaxf(raw, p.eps), 1.0f - p.eps), p.p_f32), sf);   // clamp in prob's dtype, then .to
    cur = rnd(ld1(p.hidden, int64_t(rank) * p.h_sr + d, p.h_f32), sf);
  }
  const float last = ld1(p.last, int64_t(b) * p.l_sr + d, sf);
  const float r = rnd(rnd(pb * cur, sf) + rnd(rnd(1.0f - pb, sf) * last, sf), sf);
  if (sf) {
    reinterpret_cast<float*>(p.last)[int64_t(b) * p.l_sr + d] = r;
    if (p.out) reinterpret_cast<float*>(p.out)[int64_t(b) * p.o_sr + d] = r;
  } else {
    reinterpret_cast<bf16_t*>(p.last)[int64_t(b) * p.l_sr + d] = f2bf(r);
    if (p.out) reinterpret_cast<bf16_t*>(p.out)[int64_t(b) * p.o_sr + d] = f2bf(r);
  }
}

// ------------------------------------------------------------------------------------------------
// host side
// ------------------------------------------------------------------------------------------------
static int es_of(int dt) { return dt == MOTE_F32 ? 4 : 2; }
static bool dt_ok2(int dt) { return dt == MOTE_F32 || dt == MOTE_BF16; }

int launch_chunk_route(const mote_chunk_route_args* a, hipStream_t stream) {
  if (!a) return set_error(MOTE_ERR_ARGUMENT, "chunk_route: null args");
  if (a->B < 0 || a->L < 0) return set_error(MOTE_ERR_SHAPE, "chunk_route: B = %d, L = %d", a->B, a->L);
  if (a->B == 0) return MOTE_OK;
  if (!a->num || (a->L > 0 && (!a->mask || !a->cum || !a->perm)))
    return set_error(MOTE_ERR_ARGUMENT, "chunk_route: null pointer");
  RouteParams p;
  p.mask = a->mask; p.mask_sr = a->mask_sr; p.cum = a->cum; p.perm = a->perm; p.num = a->num; p.L = a->L;
  p.vec = reinterpret_cast<uintptr_t>(a->mask) % 16 == 0 && a->mask_sr % 16 == 0;
  p.vec4 = reinterpret_cast<uintptr_t>(a->cum) % 16 == 0 && a->L % 4 == 0;
  p.vecp = reinterpret_cast<uintptr_t>(a->perm) % 16 == 0 && a->L % 4 == 0;
  const bool cu_here = a->B == 1 && a->L <= kRouteThreads * kRoutePer;
  p.cu = cu_here ? a->cu_seqlens : nullptr;
  hipLaunchKernelGGL(chunk_route_kernel, dim3(a->B), dim3(kRouteThreads), 0, stream, p);
  int rc = check_launch("chunk_route");
  if (rc || !a->cu_seqlens || cu_here) return rc;
  hipLaunchKernelGGL(chunk_cu_kernel, dim3(1), dim3(kRouteThreads), 0, stream, a->num, a->B, a->cu_seqlens);
  return check_launch("chunk_route/cu_seqlens");
}

static int gather_common(const char* what, int dtype, int D, const void* s, int64_t s_sb, int64_t s_sr, void* d,
                         int64_t d_sb, int64_t d_sr, GatherParams& p) {
  if (!dt_ok2(dtype)) return set_error(MOTE_ERR_ARGUMENT, "%s: bad dtype", what);
  const int es = es_of(dtype);
  if (D <= 0 || (D * es) % 16) return set_error(MOTE_ERR_SHAPE, "%s: D = %d (rows must be whole 16-byte units)", what, D);
  if (reinterpret_cast<uintptr_t>(s) % 16 || reinterpret_cast<uintptr_t>(d) % 16 || (s_sb * es) % 16 ||
      (s_sr * es) % 16 || (d_sb * es) % 16 || (d_sr * es) % 16)
    return set_error(MOTE_ERR_ARGUMENT, "%s: rows must start on 16-byte boundaries", what);
  p.src = reinterpret_cast<const uint8_t*>(s); p.s_sb = s_sb * es; p.s_sr = s_sr * es;
  p.dst = reinterpret_cast<uint8_t*>(d); p.d_sb = d_sb * es; p.d_sr = d_sr * es;
  p.row_units = D * es / 16;
  return MOTE_OK;
}

int launch_chunk_gather(const mote_chunk_gather_args* a, hipStream_t stream) {
  if (!a) return set_error(MOTE_ERR_ARGUMENT, "chunk_gather: null args");
  if (a->B < 0 || a->L < 0 || a->M < 0 || a->M > a->L)
    return set_error(MOTE_ERR_SHAPE, "chunk_gather: B = %d, L = %d, M = %d (need 0 <= M <= L)", a->B, a->L, a->M);
  if (int64_t(a->B) * a->M == 0) return MOTE_OK;
  if (!a->hidden || !a->out || !a->perm || (a->cu_seqlens && !a->num))
    return set_error(MOTE_ERR_ARGUMENT, "chunk_gather: null pointer");
  GatherParams p = {};
  int rc = gather_common("chunk_gather", a->dtype, a->D, a->hidden, a->h_sb, a->h_sr, a->out, a->o_sb, a->o_sr, p);
  if (rc) return rc;
  p.perm = a->perm; p.num = a->num; p.cu = a->cu_seqlens; p.B = a->B; p.L = a->L; p.M = a->M;
  const int64_t rows = int64_t(a->B) * a->M;
  hipLaunchKernelGGL(chunk_gather_kernel, dim3(unsigned((rows + 3) / 4)), dim3(256), 0, stream, p);
  return check_launch("chunk_gather");
}

int launch_chunk_gather_bwd(const mote_chunk_gather_bwd_args* a, hipStream_t stream) {
  if (!a) return set_error(MOTE_ERR_ARGUMENT, "chunk_gather_bwd: null args");
  if (a->B < 0 || a->L < 0 || a->M < 0 || a->M > a->L)
    return set_error(MOTE_ERR_SHAPE, "chunk_gather_bwd: B = %d, L = %d, M = %d", a->B, a->L, a->M);
  if (int64_t(a->B) * a->L == 0) return MOTE_OK;
  if (!a->dhidden || !a->mask || !a->cum || !a->num || (a->M > 0 && !a->dout))
    return set_error(MOTE_ERR_ARGUMENT, "chunk_gather_bwd: null pointer");
  GatherParams p = {};
  const void* src = a->dout ? a->dout : a->dhidden;  // M == 0: nothing is read
  int rc = gather_common("chunk_gather_bwd", a->dtype, a->D, src, a->g_sb, a->g_sr, a->dhidden, a->dh_sb, a->dh_sr, p);
  if (rc) return rc;
  p.num = a->num; p.cu = a->cu_seqlens; p.mask = a->mask; p.mask_sr = a->mask_sr; p.cum = a->cum;
  p.B = a->B; p.L = a->L; p.M = a->M;
  const int64_t rows = int64_t(a->B) * a->L;
  hipLaunchKernelGGL(chunk_gather_bwd_kernel, dim3(unsigned((rows + 3) / 4)), dim3(256), 0, stream, p);
  return check_launch("chunk_gather_bwd");
}

// segments per row: the chunk rows in fixed segments of kDcSeg
static int dc_nseg(int M) { return M > 0 ? (M + kDcSeg - 1) / kDcSeg : 1; }

static int dc_check(const char* what, int B, int L, int M, int D) {
  if (B < 0 || L < 0 || M < 0 || M > L || D <= 0 || D % 2)
    return set_error(MOTE_ERR_SHAPE, "%s: B = %d, L = %d, M = %d, D = %d (need M <= L, D even)", what, B, L, M, D);
  if (B > 65535 || dc_nseg(M) > 65535)  // grid y / z limits
    return set_error(MOTE_ERR_SHAPE, "%s: B = %d, M = %d too large for one launch", what, B, M);
  return MOTE_OK;
}

// segments and workgroups of segments per row
static int dc_ngrp(int M) { return (dc_nseg(M) + kDcGrp - 1) / kDcGrp; }

// floats of a workspace piece, rounded up so the next piece starts on a 256-byte boundary
static size_t dc_piece(size_t floats) { return (floats + 63) / 64 * 64; }

// forward workspace: the workgroup aggregates (values [B, ngrp, D], decays [B, ngrp]), chunk p [B, M],
// the segment aggregates (values [B, nseg, D], decays [B, nseg])
size_t dechunk_workspace_bytes(const mote_dechunk_args* a) {
  if (a->B <= 0 || a->D <= 0) return 0;
  const size_t ng = size_t(a->B) * dc_ngrp(a->M);
  const size_t ns = ng * kDcGrp;
  return (dc_piece(ng * a->D) + dc_piece(ng) + dc_piece(size_t(a->B) * a->M) + dc_piece(ns * a->D) + dc_piece(ns)) *
         sizeof(float);
}

// backward workspace: segment and workgroup aggregates, chunk p, dp partials, ds rows
size_t dechunk_bwd_workspace_bytes(const mote_dechunk_bwd_args* a) {
  if (a->B <= 0 || a->D <= 0) return 0;
  const size_t ng = size_t(a->B) * dc_ngrp(a->M), ns = ng * kDcGrp;
  const size_t strips = (a->D + kFsCh - 1) / kFsCh;  // the narrower strips of the two paths
  return (dc_piece(ns * a->D) + dc_piece(ns) + dc_piece(ng * a->D) + dc_piece(ng) + dc_piece(size_t(a->B) * a->M) +
          dc_piece(size_t(a->B) * strips * a->M) + dc_piece(size_t(a->B) * a->M * a->D)) *
         sizeof(float);
}

// 16-byte rows: the vector path's condition for one tensor (elements of es bytes)
static bool al16(const void* ptr, int64_t sb, int64_t sr, int es) {
  return ptr == nullptr || (reinterpret_cast<uintptr_t>(ptr) % 16 == 0 && (sb * es) % 16 == 0 && (sr * es) % 16 == 0);
}

// 2-element accesses: the pointer aligned to two elements, even strides
static bool al_el(const void* ptr, int64_t sb, int64_t sr, int es) {
  return ptr == nullptr || (reinterpret_cast<uintptr_t>(ptr) % (2 * es) == 0 && sb % 2 == 0 && sr % 2 == 0);
}

int launch_dechunk_fwd(const mote_dechunk_args* a, hipStream_t stream) {
  if (!a) return set_error(MOTE_ERR_ARGUMENT, "dechunk_fwd: null args");
  int rc = dc_check("dechunk_fwd", a->B, a->L, a->M, a->D);
  if (rc) return rc;
  if (!dt_ok2(a->dtype) || !dt_ok2(a->prob_dtype) || a->out_dtype != a->dtype)
    return set_error(MOTE_ERR_ARGUMENT, "dechunk_fwd: bad dtype (out_dtype must equal dtype)");
  if (a->M == 0 && !a->init)
    return set_error(MOTE_ERR_SHAPE, "dechunk_fwd: no chunks and no carried value (nothing to expand)");
  if (int64_t(a->B) * a->L == 0) return MOTE_OK;
  if (!a->prob || !a->num || !a->perm || !a->cum || !a->out || (a->M > 0 && !a->hidden))
    return set_error(MOTE_ERR_ARGUMENT, "dechunk_fwd: null pointer");
  if (!al_el(a->hidden, a->h_sb, a->h_sr, es_of(a->dtype)) || !al_el(a->out, a->o_sb, a->o_sr, es_of(a->dtype)) ||
      reinterpret_cast<uintptr_t>(a->init) % 8 || reinterpret_cast<uintptr_t>(a->w) % 8)
    return set_error(MOTE_ERR_ARGUMENT, "dechunk_fwd: rows must start on 2-element boundaries");
  if (!a->workspace || a->workspace_bytes < dechunk_workspace_bytes(a))
    return set_error(MOTE_ERR_WORKSPACE, "dechunk_fwd: workspace too small");
  DechunkParams p = {};
  p.x = a->hidden; p.x_sb = a->h_sb; p.x_sr = a->h_sr; p.prob = a->prob; p.p_sb = a->p_sb; p.p_sr = a->p_sr;
  p.perm = a->perm; p.num = a->num; p.cum = a->cum; p.init = a->init; p.out = a->out; p.o_sb = a->o_sb; p.o_sr = a->o_sr;
  p.w = a->w; p.B = a->B; p.L = a->L; p.M = a->M; p.D = a->D; p.eps = a->eps;
  p.p_f32 = a->prob_dtype == MOTE_F32;
  p.ngrp = dc_ngrp(a->M);
  p.nseg = p.ngrp * kDcGrp;
  p.nstrips = (a->D + kDcCh - 1) / kDcCh;
  p.grpv = reinterpret_cast<float*>(a->workspace);
  p.grpd = p.grpv + dc_piece(size_t(a->B) * p.ngrp * a->D);
  p.pc = p.grpd + dc_piece(size_t(a->B) * p.ngrp);
  p.segv = p.pc + dc_piece(size_t(a->B) * a->M);
  p.segd = p.segv + dc_piece(size_t(a->B) * p.nseg * a->D);
  const dim3 grid(p.nstrips, p.ngrp, a->B);
  const dim3 block(64 * kDcGrp);
  const int es = es_of(a->dtype);
  const bool vec = a->D % 8 == 0 && al16(a->hidden, a->h_sb, a->h_sr, es) && al16(a->out, a->o_sb, a->o_sr, es) &&
                   reinterpret_cast<uintptr_t>(a->init) % 16 == 0 && reinterpret_cast<uintptr_t>(a->w) % 16 == 0;
  if (vec) {  // 64-channel strips
    DechunkParams f = p;
    f.nstrips = (a->D + kFsCh - 1) / kFsCh;
    const dim3 g1(f.nstrips, f.ngrp, a->B), g2(f.nstrips, f.nseg, a->B);
    if (a->dtype == MOTE_F32) hipLaunchKernelGGL(dechunk_grp_w_kernel<true>, g1, dim3(64 * kDcGrp), 0, stream, f);
    else hipLaunchKernelGGL(dechunk_grp_w_kernel<false>, g1, dim3(64 * kDcGrp), 0, stream, f);
    rc = check_launch("dechunk_fwd/segments");
    if (rc) return rc;
    if (a->dtype == MOTE_F32) hipLaunchKernelGGL(dechunk_out_w_kernel<true>, g2, dim3(64), 0, stream, f);
    else hipLaunchKernelGGL(dechunk_out_w_kernel<false>, g2, dim3(64), 0, stream, f);
    return check_launch("dechunk_fwd/scan");
  }
  if (a->dtype == MOTE_F32) {
    hipLaunchKernelGGL(dechunk_grp_kernel<true>, grid, block, 0, stream, p);
    rc = check_launch("dechunk_fwd/segments");
    if (rc) return rc;
    hipLaunchKernelGGL(dechunk_out_kernel<true>, grid, block, 0, stream, p);
  } else {
    hipLaunchKernelGGL(dechunk_grp_kernel<false>, grid, block, 0, stream, p);
    rc = check_launch("dechunk_fwd/segments");
    if (rc) return rc;
    hipLaunchKernelGGL(dechunk_out_kernel<false>, grid, block, 0, stream, p);
  }
  return check_launch("dechunk_fwd/scan");
}

int launch_dechunk_bwd(const mote_dechunk_bwd_args* a, hipStream_t stream) {
  if (!a) return set_error(MOTE_ERR_ARGUMENT, "dechunk_bwd: null args");
  int rc = dc_check("dechunk_bwd", a->B, a->L, a->M, a->D);
  if (rc) return rc;
  if (!dt_ok2(a->dtype) || !dt_ok2(a->prob_dtype) || a->dout_dtype != a->dtype || a->dx_dtype != a->dtype ||
      !dt_ok2(a->dprob_dtype))
    return set_error(MOTE_ERR_ARGUMENT, "dechunk_bwd: bad dtype (dout and dhidden in hidden's dtype)");
  if (a->M == 0) return set_error(MOTE_ERR_SHAPE, "dechunk_bwd: no chunks");
  if (int64_t(a->B) * a->L == 0) return MOTE_OK;
  if (!a->dout || !a->hidden || !a->prob || !a->perm || !a->num || !a->mask || !a->cum || !a->w || !a->dhidden ||
      !a->dprob)
    return set_error(MOTE_ERR_ARGUMENT, "dechunk_bwd: null pointer");
  const int es = es_of(a->dtype);
  if (!al_el(a->dout, a->g_sb, a->g_sr, es) || !al_el(a->dhidden, a->dh_sb, a->dh_sr, es) ||
      reinterpret_cast<uintptr_t>(a->w) % 8)
    return set_error(MOTE_ERR_ARGUMENT, "dechunk_bwd: rows must start on 2-element boundaries");
  if (!a->workspace || a->workspace_bytes < dechunk_bwd_workspace_bytes(a))
    return set_error(MOTE_ERR_WORKSPACE, "dechunk_bwd: workspace too small");
  DechunkParams p = {};
  p.x = a->hidden; p.x_sb = a->h_sb; p.x_sr = a->h_sr; p.prob = a->prob; p.p_sb = a->p_sb; p.p_sr = a->p_sr;
  p.perm = a->perm; p.num = a->num; p.cum = a->cum; p.init = nullptr; p.w = const_cast<float*>(a->w);
  p.dout = a->dout; p.g_sb = a->g_sb; p.g_sr = a->g_sr; p.dx = a->dhidden; p.dx_sb = a->dh_sb; p.dx_sr = a->dh_sr;
  p.B = a->B; p.L = a->L; p.M = a->M; p.D = a->D; p.eps = a->eps;
  p.p_f32 = a->prob_dtype == MOTE_F32;
  p.ngrp = dc_ngrp(a->M);
  p.nseg = p.ngrp * kDcGrp;
  p.nstrips = (a->D + kDcCh - 1) / kDcCh;
  const size_t ns = size_t(a->B) * p.nseg, ng = size_t(a->B) * p.ngrp;
  p.segv = reinterpret_cast<float*>(a->workspace);
  p.segd = p.segv + dc_piece(ns * a->D);
  p.grpv = p.segd + dc_piece(ns);
  p.grpd = p.grpv + dc_piece(ng * a->D);
  p.pc = p.grpd + dc_piece(ng);
  p.part = p.pc + dc_piece(size_t(a->B) * a->M);
  p.ds = p.part + dc_piece(size_t(a->B) * ((a->D + kFsCh - 1) / kFsCh) * a->M);  // 256-byte aligned
  const dim3 grid(p.nstrips, p.ngrp, a->B);
  const dim3 block(64 * kDcGrp);
  const int64_t crows = int64_t(a->B) * a->M;
  const int vec = (a->D % 8) == 0 && reinterpret_cast<uintptr_t>(a->dout) % 16 == 0 && (a->g_sb * es) % 16 == 0 &&
                  (a->g_sr * es) % 16 == 0 && reinterpret_cast<uintptr_t>(p.ds) % 16 == 0;
  const bool vg = a->D % 8 == 0 && a->D <= kFsMaxStrips * kFsCh && al16(a->dhidden, a->dh_sb, a->dh_sr, es) &&
                  reinterpret_cast<uintptr_t>(a->w) % 16 == 0;
  p.dprob = a->dprob; p.dp_sb = a->dp_sb; p.dp_sr = a->dp_sr; p.dp_f32 = a->dprob_dtype == MOTE_F32;
  if (vec && vg) {  // balanced chunk sums, then the scan over 64-channel strips
    const dim3 dgrid(unsigned((a->L + kDsBytes - 1) / kDsBytes), a->B);
    if (a->dtype == MOTE_F32) hipLaunchKernelGGL(dechunk_dsum_bal_kernel<true>, dgrid, dim3(64), 0, stream, p);
    else hipLaunchKernelGGL(dechunk_dsum_bal_kernel<false>, dgrid, dim3(64), 0, stream, p);
    rc = check_launch("dechunk_bwd/chunk sums");
    if (rc) return rc;
    DechunkParams f = p;
    f.nstrips = (a->D + kFsCh - 1) / kFsCh;
    hipLaunchKernelGGL(dechunk_bwd_grp_w_kernel, dim3(f.nstrips, f.ngrp, a->B), dim3(64 * kDcGrp), 0, stream, f);
    rc = check_launch("dechunk_bwd/segments");
    if (rc) return rc;
    const dim3 sgrid(f.nseg, a->B), sblock(64 * f.nstrips);
    if (a->dtype == MOTE_F32) hipLaunchKernelGGL(dechunk_bwd_out_w_kernel<true>, sgrid, sblock, 0, stream, f);
    else hipLaunchKernelGGL(dechunk_bwd_out_w_kernel<false>, sgrid, sblock, 0, stream, f);
    return check_launch("dechunk_bwd");
  }
  if (a->dtype == MOTE_F32)
    hipLaunchKernelGGL(dechunk_dsum_kernel<true>, dim3(unsigned((crows + 3) / 4)), dim3(256), 0, stream, p, vec);
  else
    hipLaunchKernelGGL(dechunk_dsum_kernel<false>, dim3(unsigned((crows + 3) / 4)), dim3(256), 0, stream, p, vec);
  rc = check_launch("dechunk_bwd/byte sums");
  if (rc) return rc;
  hipLaunchKernelGGL(dechunk_bwd_grp_kernel, grid, block, 0, stream, p);
  rc = check_launch("dechunk_bwd/segments");
  if (rc) return rc;
  if (a->dtype == MOTE_F32) hipLaunchKernelGGL(dechunk_bwd_out_kernel<true>, grid, block, 0, stream, p);
  else hipLaunchKernelGGL(dechunk_bwd_out_kernel<false>, grid, block, 0, stream, p);
  rc = check_launch("dechunk_bwd");
  if (rc) return rc;
  const int64_t n = int64_t(a->B) * a->L;
  hipLaunchKernelGGL(dechunk_dprob_kernel, dim3(unsigned((n + 255) / 256)), dim3(256), 0, stream, p, a->mask,
                     a->mask_sr, a->cum, a->dprob, a->dp_sb, a->dp_sr, int(a->dprob_dtype == MOTE_F32));
  return check_launch("dechunk_bwd/dprob");
}

int launch_dechunk_step(const mote_dechunk_step_args* a, hipStream_t stream) {
  if (!a) return set_error(MOTE_ERR_ARGUMENT, "dechunk_step: null args");
  if (a->B < 0 || a->D <= 0) return set_error(MOTE_ERR_SHAPE, "dechunk_step: B = %d, D = %d", a->B, a->D);
  if (!dt_ok2(a->prob_dtype) || !dt_ok2(a->hidden_dtype) || !dt_ok2(a->state_dtype))
    return set_error(MOTE_ERR_ARGUMENT, "dechunk_step: bad dtype");
  if (a->B == 0) return MOTE_OK;
  if (!a->mask || !a->prob || !a->last_value) return set_error(MOTE_ERR_ARGUMENT, "dechunk_step: null pointer");
  DcStepParams p;
  p.mask = a->mask; p.prob = a->prob; p.p_sr = a->p_sr; p.hidden = a->hidden; p.h_sr = a->h_sr;
  p.last = a->last_value; p.l_sr = a->l_sr; p.out = a->out; p.o_sr = a->o_sr;
  p.B = a->B; p.D = a->D; p.eps = a->eps;
  p.p_f32 = a->prob_dtype == MOTE_F32; p.h_f32 = a->hidden_dtype == MOTE_F32; p.s_f32 = a->state_dtype == MOTE_F32;
  hipLaunchKernelGGL(dechunk_step_kernel, dim3((a->D + 255) / 256, a->B), dim3(256), 0, stream, p);
  return check_launch("dechunk_step");
}

}  // namespace mote
