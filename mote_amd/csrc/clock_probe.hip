// mote_clock_probe: the shader clock of the GPU at the moment of the launch. Each workgroup's first
// wave reads the shader-clock counter (s_memtime) and the constant 100 MHz counter (s_memrealtime)
// before and after a short loop of matrix-core products and exponentials; the clock is the ratio of
// the two counts times 100 MHz, with no host timing involved. Launched between the kernels of a timed
// run it reads the clock those kernels ran at (the clock follows the load on a scale of milliseconds),
// so a compute-bound timing can be quoted with the clock it ran at and compared across machines.
#include "common.hpp"
#include "params.hpp"

namespace mote {

__global__ void __launch_bounds__(256) clock_probe_kernel(int64_t* out, int iters) {
  using E = Elem<bf16_t>;
  E::Frag a, b;
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    a.v[i] = (__bf16)(1e-3f * float(threadIdx.x + i));
    b.v[i] = (__bf16)(1e-3f * float(i));
  }
  f32x4 c0{}, c1{};
  float e[4] = {1e-3f * threadIdx.x, 0.25f, 0.5f, 0.75f};
  const int64_t r0 = __builtin_amdgcn_s_memrealtime();
  const int64_t t0 = __builtin_amdgcn_s_memtime();
  for (int it = 0; it < iters; ++it) {
    c0 = E::mma(a, b, c0);
#pragma unroll
    for (int k = 0; k < 4; ++k) e[k] = fexp2(e[k] * -0.5f);
    c1 = E::mma(b, a, c1);
  }
  const int64_t t1 = __builtin_amdgcn_s_memtime();
  const int64_t r1 = __builtin_amdgcn_s_memrealtime();
  const float s = c0[0] + c1[1] + e[0] + e[1] + e[2] + e[3];
  if (threadIdx.x == 0) {
    out[3 * blockIdx.x] = t1 - t0;
    out[3 * blockIdx.x + 1] = r1 - r0;
    out[3 * blockIdx.x + 2] = (int64_t)__float_as_int(s);  // keeps the loop's work alive
  }
}

}  // namespace mote

extern "C" int mote_clock_probe(int64_t* out, int workgroups, int iters, void* stream) {
  if (!out || workgroups <= 0 || iters <= 0)
    return mote::set_error(MOTE_ERR_ARGUMENT, "mote_clock_probe: out needs 3 x %d int64, iters > 0", workgroups);
  hipLaunchKernelGGL(mote::clock_probe_kernel, dim3(workgroups), dim3(256), 0,
                     reinterpret_cast<hipStream_t>(stream), out, iters);
  return mote::check_launch("mote_clock_probe");
}
