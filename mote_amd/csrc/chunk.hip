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
// arithmetic) of one segment. Phase 1 runs each segment from zero and keeps its end value e_s and decay
// A_s = prod (1 - p). Phase 2 folds the earlier segments' (A, e) into the carry in order, runs the
// segment again from it, keeps z (fp32, for the backward) and writes z_m to every byte of chunk m, i.e. bytes
// [perm[m], perm[m + 1]) (the last chunk to L): out[t] = z[cum[t] - 1] as dc.py:329-335 gathers it.
// The segment size is fixed, so the arithmetic that produces z_m depends on chunks <= m only: the
// result is causal bit for bit, as the reference keeps its own (dc.py:265-268).
// The backward mirrors this with a reverse scan g_m = ds_m + (1 - p_{m+1}) g_{m+1}, ds_m the sum of
// the output gradient over chunk m's bytes; dx_m = p_m g_m, dp_m = sum_d g_m (x_m - z_{m-1}) (a
// fixed-order sum over channel strips), scattered to boundary_prob[..., 1] through the clamp.
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
  int L, vec, vec4;                // vec: mask rows on 16-byte boundaries; vec4: cum rows too
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
      if (t < p.L) perm[f[k] ? run - 1 : n + t - run] = t;
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

struct DechunkParams {
  const void* x; int64_t x_sb, x_sr;        // hidden [B, M, D] (elements)
  const void* prob; int64_t p_sb, p_sr;     // boundary_prob [B, L, 2] (elements; p at +1)
  const int32_t* perm; const int32_t* num;
  const float* init;                        // [B, D] carried value, or null
  void* out; int64_t o_sb, o_sr;            // [B, L, D] (forward)
  float* w;                                 // [B, M, D] fp32: x_m - z_{m-1}, kept for the backward (may be null)
  const void* dout; int64_t g_sb, g_sr;     // [B, L, D] (backward)
  void* dx; int64_t dx_sb, dx_sr;           // [B, M, D] (backward)
  float* ds;                                // [B, M, D] fp32: dout summed over each chunk's bytes (backward)
  void* zc;                                 // [B, M + 1, D] hidden's dtype: carried value, then z_m (forward)
  float* segv; float* segd;                 // [B, nseg, D] segment values, [B, nseg] segment decays
  float* part;                              // [B, nstrips, M] dp partials (backward)
  int B, L, M, D, nseg, nstrips, p_f32;
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

// phase 1 (forward): segment run from zero -> end value and decay. The segment's x rows are loaded
// up front (clamped, unconditional), so one memory latency covers the 64 steps.
template <bool F32>
__global__ void __launch_bounds__(64) dechunk_seg_kernel(const DechunkParams p) {
  typedef Pair<F32> P;
  const int lane = threadIdx.x, strip = blockIdx.x, s = blockIdx.y, b = blockIdx.z;
  const int d = min(strip * kDcCh + 2 * lane, p.D - 2);
  const int n = dc_used(p, b);
  const int m0 = min(s * kDcSeg, n), cnt = min(kDcSeg, n - m0);
  float2 z = make_float2(0.f, 0.f);
  float A = 1.f;
  if (cnt > 0) {
    const float pv = dc_p(p, b, m0 + min(lane, cnt - 1));
    typename P::T xr[kDcSeg];
    const int64_t xb = b * p.x_sb + d;
#pragma unroll
    for (int i = 0; i < kDcSeg; ++i) xr[i] = P::ld(p.x, xb + int64_t(m0 + min(i, cnt - 1)) * p.x_sr);
#pragma unroll
    for (int i = 0; i < kDcSeg; ++i) {
      const float pc = i < cnt ? rdl(pv, i) : 0.f;  // past the segment: p = 0 leaves z and A as they are
      const float a = 1.f - pc;
      const float2 x = P::cvt(xr[i]);
      z.x = fmaf(a, z.x, pc * x.x);
      z.y = fmaf(a, z.y, pc * x.y);
      A *= a;
    }
  }
  const int64_t si = int64_t(b) * p.nseg + s;
  if (strip * kDcCh + 2 * lane < p.D) stf2(p.segv, si * p.D + d, z);
  if (strip == 0 && lane == 0) p.segd[si] = A;
}

// c <- A_j c + e_j for j = 0 .. s-1 (in order), in batches of 16 segments, the next batch loading while
// the current one folds
__device__ __forceinline__ void dc_fold_fwd(const DechunkParams& p, int b, int d, int s, float2& c) {
  const int64_t sb0 = int64_t(b) * p.nseg;
  float2 ea[16], eb[16];
  float Aa[16], Ab[16];
  auto load = [&](float2 (&e)[16], float (&A)[16], int j0) {
#pragma unroll
    for (int k = 0; k < 16; ++k) {
      const int j = max(min(j0 + k, s - 1), 0);
      e[k] = ldf2(p.segv, (sb0 + j) * p.D + d);
      A[k] = p.segd[sb0 + j];
    }
  };
  auto fold = [&](float2 (&e)[16], float (&A)[16], int j0) {
#pragma unroll
    for (int k = 0; k < 16; ++k) {
      if (j0 + k < s) {
        c.x = fmaf(A[k], c.x, e[k].x);
        c.y = fmaf(A[k], c.y, e[k].y);
      }
    }
  };
  if (s <= 0) return;
  load(ea, Aa, 0);
  for (int j0 = 0; j0 < s; j0 += 32) {
    load(eb, Ab, j0 + 16);
    fold(ea, Aa, j0);
    if (j0 + 16 >= s) break;
    load(ea, Aa, j0 + 32);
    fold(eb, Ab, j0 + 16);
  }
}

// G <- f_j + A'_j G for j = last .. s+1 (from the row's last segment down), batched as dc_fold_fwd
__device__ __forceinline__ void dc_fold_bwd(const DechunkParams& p, int b, int d, int s, int last, float2& G) {
  const int64_t sb0 = int64_t(b) * p.nseg;
  float2 fa[16], fb[16];
  float Aa[16], Ab[16];
  auto load = [&](float2 (&f)[16], float (&A)[16], int j1) {
#pragma unroll
    for (int k = 0; k < 16; ++k) {
      const int j = min(max(j1 - k, s + 1), last);
      f[k] = ldf2(p.segv, (sb0 + j) * p.D + d);
      A[k] = p.segd[sb0 + j];
    }
  };
  auto fold = [&](float2 (&f)[16], float (&A)[16], int j1) {
#pragma unroll
    for (int k = 0; k < 16; ++k) {
      if (j1 - k > s) {
        G.x = fmaf(A[k], G.x, f[k].x);
        G.y = fmaf(A[k], G.y, f[k].y);
      }
    }
  };
  if (last <= s) return;
  load(fa, Aa, last);
  for (int j1 = last; j1 > s; j1 -= 32) {
    load(fb, Ab, j1 - 16);
    fold(fa, Aa, j1);
    if (j1 - 16 <= s) break;
    load(fa, Aa, j1 - 32);
    fold(fb, Ab, j1 - 16);
  }
}

// phase 2 (forward): carry in, run again; keep w_m = x_m - z_{m-1} (fp32) and the compact values
// zc[b, 1 + m] = z_m in hidden's dtype, with zc[b, 0] = the carried value (or 0)
template <bool F32>
__global__ void __launch_bounds__(64) dechunk_scan_kernel(const DechunkParams p) {
  typedef Pair<F32> P;
  const int lane = threadIdx.x, strip = blockIdx.x, s = blockIdx.y, b = blockIdx.z;
  const bool live = strip * kDcCh + 2 * lane < p.D;
  const int d = min(strip * kDcCh + 2 * lane, p.D - 2);
  const int n = dc_used(p, b);
  const int m0 = min(s * kDcSeg, n), cnt = min(kDcSeg, n - m0);
  float2 c = make_float2(0.f, 0.f);
  if (p.init) c = ldf2(p.init, int64_t(b) * p.D + d);
  const int64_t zb = int64_t(b) * (p.M + 1) * p.D + d;
  if (s == 0 && live) P::st(p.zc, zb, c);
  if (cnt <= 0) return;
  const float pv = dc_p(p, b, m0 + min(lane, cnt - 1));
  typename P::T xr[kDcSeg];
  const int64_t xb = b * p.x_sb + d;
#pragma unroll
  for (int i = 0; i < kDcSeg; ++i) xr[i] = P::ld(p.x, xb + int64_t(m0 + min(i, cnt - 1)) * p.x_sr);
  dc_fold_fwd(p, b, d, s, c);  // c <- A_j c + e_j, j = 0 .. s-1, in order
  float2 z = c;
  float* wrow = p.w + (int64_t(b) * p.M + m0) * p.D + d;
  void* zrow = reinterpret_cast<uint8_t*>(p.zc) + (zb + int64_t(m0 + 1) * p.D) * (F32 ? 4 : 2);
#pragma unroll
  for (int i = 0; i < kDcSeg; ++i) {
    if (i < cnt) {
      const float pc = rdl(pv, i), a = 1.f - pc;
      const float2 x = P::cvt(xr[i]);
      if (live && p.w) stf2(wrow, int64_t(i) * p.D, make_float2(x.x - z.x, x.y - z.y));
      z.x = fmaf(a, z.x, pc * x.x);
      z.y = fmaf(a, z.y, pc * x.y);
      if (live) P::st(zrow, int64_t(i) * p.D, z);
    }
  }
}

// out[b, t] = zc[b, cum[t]] with the carried value, zc[b, max(cum[t], 1)] without (bytes before the
// first boundary read chunk 0, dc.py:326): one wave per byte row, 16-byte units when rows allow
__global__ void __launch_bounds__(256) dechunk_expand_kernel(const DechunkParams p, const int32_t* cum, int es,
                                                             int vec) {
  const int lane = threadIdx.x & 63;
  const int64_t r = int64_t(blockIdx.x) * 4 + (threadIdx.x >> 6);
  if (r >= int64_t(p.B) * p.L) return;
  const int b = int(r / p.L), t = int(r % p.L);
  const int c = cum[int64_t(b) * p.L + t];
  const int idx = p.init ? min(c, p.M) : max(min(c, p.M), 1);
  const uint8_t* src = reinterpret_cast<const uint8_t*>(p.zc) + ((int64_t(b) * (p.M + 1) + idx) * p.D) * es;
  uint8_t* dst = reinterpret_cast<uint8_t*>(p.out) + (b * p.o_sb + int64_t(t) * p.o_sr) * es;
  const int bytes = p.D * es;
  if (vec) {
    for (int u = lane; u < bytes / 16; u += 64)
      reinterpret_cast<uint4*>(dst)[u] = reinterpret_cast<const uint4*>(src)[u];
  } else {
    for (int u = lane; u < bytes / 4; u += 64)
      reinterpret_cast<uint32_t*>(dst)[u] = reinterpret_cast<const uint32_t*>(src)[u];
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
  const int n = dc_used(p, b);
  if (m >= n) return;
  const int t0 = dc_lo(p, b, m, n), t1 = dc_lo(p, b, m + 1, n);
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

// phase 1 (backward): reverse scan of a segment from zero over its ds rows (loaded up front):
// h_m = ds_m + (1 - p_{m+1}) h_{m+1}. Keeps the value at the first chunk and the decay
// prod_{k = m0+1}^{m1} (1 - p_k) that carries the next segment's value into it.
__global__ void __launch_bounds__(64) dechunk_bwd_seg_kernel(const DechunkParams p) {
  const int lane = threadIdx.x, strip = blockIdx.x, s = blockIdx.y, b = blockIdx.z;
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
  if (strip * kDcCh + 2 * lane < p.D) stf2(p.segv, si * p.D + d, h);
  if (strip == 0 && lane == 0) p.segd[si] = A;
}

// phase 2 (backward): carry from the later segments, reverse run again over ds; dx = p g and the dp
// partials sum_d g (x - z_prev) = sum_d g w, reduced over the wave's channels in a fixed order.
// ds and w rows come in 4 stages of 16 chunks, the next stage loading while the current one runs.
template <bool F32>
__global__ void __launch_bounds__(64) dechunk_bwd_out_kernel(const DechunkParams p) {
  typedef Pair<F32> P;
  __shared__ float red[kDcSeg][65];
  const int lane = threadIdx.x, strip = blockIdx.x, s = blockIdx.y, b = blockIdx.z;
  const bool live = strip * kDcCh + 2 * lane < p.D;
  const int d = min(strip * kDcCh + 2 * lane, p.D - 2);
  const int n = dc_used(p, b);
  const int m0 = min(s * kDcSeg, n), cnt = min(kDcSeg, n - m0);
  const int64_t xb = b * p.dx_sb + d;
  if (s == p.nseg - 1) {  // rows no byte reads: zero gradient
    for (int m = n; m < p.M; ++m)
      if (live) P::st(p.dx, xb + int64_t(m) * p.dx_sr, make_float2(0.f, 0.f));
  }
  if (cnt <= 0) return;
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
  // G = g at chunk m0 + cnt: fold the row's segments last .. s+1 (G <- f_j + A'_j G)
  float2 g = make_float2(0.f, 0.f);
  dc_fold_bwd(p, b, d, s, (n + kDcSeg - 1) / kDcSeg - 1, g);
  auto run = [&](float2 (&dsv)[16], float2 (&wv)[16], int q) {
#pragma unroll
    for (int k = 15; k >= 0; --k) {
      const int i = 16 * q + k;
      if (i < cnt) {
        const float an = 1.f - rdl(pn, i), pc = rdl(pv, i);
        g.x = fmaf(an, g.x, dsv[k].x);
        g.y = fmaf(an, g.y, dsv[k].y);
        if (live) P::st(p.dx, xb + int64_t(m0 + i) * p.dx_sr, make_float2(pc * g.x, pc * g.y));
        red[i][lane] = live ? g.x * wv[k].x + g.y * wv[k].y : 0.f;
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
  __syncthreads();
  if (lane < cnt) {  // lane k sums chunk m0 + k over the 64 lanes, in lane order
    float a = 0.f;
    for (int l = 0; l < 64; ++l) a += red[lane][l];
    p.part[(int64_t(b) * p.nstrips + strip) * p.M + m0 + lane] = a;
  }
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

// forward workspace: zc [B, M + 1, D] in hidden's dtype (256-byte rounded), segment values and decays
static size_t dc_zc_bytes(const mote_dechunk_args* a) {
  const size_t zc = size_t(a->B) * (size_t(a->M) + 1) * a->D * es_of(a->dtype);
  return (zc + 255) / 256 * 256;
}

size_t dechunk_workspace_bytes(const mote_dechunk_args* a) {
  if (a->B <= 0 || a->D <= 0) return 0;
  const size_t nseg = dc_nseg(a->M);
  return dc_zc_bytes(a) + (size_t(a->B) * nseg * a->D + size_t(a->B) * nseg) * sizeof(float);
}

size_t dechunk_bwd_workspace_bytes(const mote_dechunk_bwd_args* a) {
  if (a->B <= 0 || a->D <= 0) return 0;
  const size_t nseg = dc_nseg(a->M);
  const size_t strips = (a->D + kDcCh - 1) / kDcCh;
  return (size_t(a->B) * nseg * a->D + size_t(a->B) * nseg + size_t(a->B) * strips * a->M +
          size_t(a->B) * a->M * a->D + 4) * sizeof(float);
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
  p.perm = a->perm; p.num = a->num; p.init = a->init; p.out = a->out; p.o_sb = a->o_sb; p.o_sr = a->o_sr;
  p.w = a->w; p.B = a->B; p.L = a->L; p.M = a->M; p.D = a->D; p.eps = a->eps;
  p.p_f32 = a->prob_dtype == MOTE_F32;
  p.nseg = dc_nseg(a->M);
  p.nstrips = (a->D + kDcCh - 1) / kDcCh;
  p.zc = a->workspace;
  p.segv = reinterpret_cast<float*>(reinterpret_cast<uint8_t*>(a->workspace) + dc_zc_bytes(a));
  p.segd = p.segv + size_t(a->B) * p.nseg * a->D;
  const dim3 grid(p.nstrips, p.nseg, a->B);
  if (a->dtype == MOTE_F32) {
    hipLaunchKernelGGL(dechunk_seg_kernel<true>, grid, dim3(64), 0, stream, p);
    rc = check_launch("dechunk_fwd/segments");
    if (rc) return rc;
    hipLaunchKernelGGL(dechunk_scan_kernel<true>, grid, dim3(64), 0, stream, p);
  } else {
    hipLaunchKernelGGL(dechunk_seg_kernel<false>, grid, dim3(64), 0, stream, p);
    rc = check_launch("dechunk_fwd/segments");
    if (rc) return rc;
    hipLaunchKernelGGL(dechunk_scan_kernel<false>, grid, dim3(64), 0, stream, p);
  }
  rc = check_launch("dechunk_fwd/scan");
  if (rc) return rc;
  const int es = es_of(a->dtype);
  const int vec = (a->D * es) % 16 == 0 && reinterpret_cast<uintptr_t>(a->out) % 16 == 0 && (a->o_sb * es) % 16 == 0 &&
                  (a->o_sr * es) % 16 == 0;
  const int64_t rows = int64_t(a->B) * a->L;
  hipLaunchKernelGGL(dechunk_expand_kernel, dim3(unsigned((rows + 3) / 4)), dim3(256), 0, stream, p, a->cum, es, vec);
  return check_launch("dechunk_fwd/expand");
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
  p.perm = a->perm; p.num = a->num; p.init = nullptr; p.w = const_cast<float*>(a->w);
  p.dout = a->dout; p.g_sb = a->g_sb; p.g_sr = a->g_sr; p.dx = a->dhidden; p.dx_sb = a->dh_sb; p.dx_sr = a->dh_sr;
  p.B = a->B; p.L = a->L; p.M = a->M; p.D = a->D; p.eps = a->eps;
  p.p_f32 = a->prob_dtype == MOTE_F32;
  p.nseg = dc_nseg(a->M);
  p.nstrips = (a->D + kDcCh - 1) / kDcCh;
  p.segv = reinterpret_cast<float*>(a->workspace);
  p.segd = p.segv + size_t(a->B) * p.nseg * a->D;
  p.part = p.segd + size_t(a->B) * p.nseg;
  // ds rows start on 16-byte boundaries (float4 accesses)
  const uintptr_t ds_at = reinterpret_cast<uintptr_t>(p.part + size_t(a->B) * p.nstrips * a->M);
  p.ds = reinterpret_cast<float*>((ds_at + 15) & ~uintptr_t(15));
  const dim3 grid(p.nstrips, p.nseg, a->B);
  const int64_t crows = int64_t(a->B) * a->M;
  const int vec = (a->D % 8) == 0 && reinterpret_cast<uintptr_t>(a->dout) % 16 == 0 && (a->g_sb * es) % 16 == 0 &&
                  (a->g_sr * es) % 16 == 0 && reinterpret_cast<uintptr_t>(p.ds) % 16 == 0;
  if (a->dtype == MOTE_F32)
    hipLaunchKernelGGL(dechunk_dsum_kernel<true>, dim3(unsigned((crows + 3) / 4)), dim3(256), 0, stream, p, vec);
  else
    hipLaunchKernelGGL(dechunk_dsum_kernel<false>, dim3(unsigned((crows + 3) / 4)), dim3(256), 0, stream, p, vec);
  rc = check_launch("dechunk_bwd/byte sums");
  if (rc) return rc;
  hipLaunchKernelGGL(dechunk_bwd_seg_kernel, grid, dim3(64), 0, stream, p);
  rc = check_launch("dechunk_bwd/segments");
  if (rc) return rc;
  if (a->dtype == MOTE_F32) hipLaunchKernelGGL(dechunk_bwd_out_kernel<true>, grid, dim3(64), 0, stream, p);
  else hipLaunchKernelGGL(dechunk_bwd_out_kernel<false>, grid, dim3(64), 0, stream, p);
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
