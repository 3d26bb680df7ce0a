// Parameter block of the Relation backward kernels (relation_bwd.hip, relation_bwd_tiles.hip).
#pragma once

#include "params.hpp"

namespace mote {

struct BwdParams {
  const void* p1; int64_t q_sb, q_sh, q_sr;
  const void* p2; int64_t k_sb, k_sh, k_sr;
  const void* info; int64_t v_sb, v_sh, v_sr;
  const void* dy; int64_t y_sb, y_sh, y_sr;
  const float* ibar;
  const float* lse;
  const float* g;
  void* dp1; int64_t dq_sb, dq_sh, dq_sr;
  void* dp2; int64_t dk_sb, dk_sh, dk_sr;
  void* dinfo; int64_t dv_sb, dv_sh, dv_sr;
  float* dlam;
  // workspace
  void* wq;      // [BH][TQp][DP]  P1 rows                      (register-staged kernels)
  void* wdib;    // [BH][TQp][DP]  dI-bar rows                  (both paths)
  void* wqT;     // [BH][DP][TQp]  P1 transposed                (register-staged kernels)
  void* wdibT;   // [BH][DP][TQp]  dI-bar transposed            (register-staged kernels)
  float* lse2;   // [BH][TQp]                                   (register-staged kernels)
  float* cvec;   // [BH][TQp]      dA - Delta                   (register-staged kernels)
  float* stat;   // [BH][TQp / 64][128]: lse2 of the block's 64 rows, then c = dA - Delta (tile kernels)
  float* duii;   // [BH][TQp]
  float* dp1acc; // [BH][TQ][D]                                 (register-staged kernels)
  float* dlam_part;  // [BH][TQp / 64]
  void* dut;     // [BH][npairs][4 waves][2 query tiles][64 lanes][8] bf16: dU as the key kernel's waves hold it (tile kernels)
  int64_t npairs;    // (query block, key block) pairs per (batch, head), PairTable::total
  int* kvq;      // control words of the fused key + query launch, or null: the two launches (tile kernels)
  int kvq_nq;    // its queues: 8, 4, 2 or 1, dividing B H
  int kvq_spin;  // polls before a query job's wait gives up (kKvqSpinLimit)
  int kvq_extra; // added to every wait's target: 0 (a test of the give-up path sets 1: never reached)
  int B, H, TQ, TK, D, q_start, TQp;
  float scale, tau_inv;
};

constexpr int kRowBlock = 64;  // rows per workgroup in the rows stage; also TQp's granularity

// Layout of the fused key + query launch's control words (BwdParams::kvq, cleared by the rows stage
// with agent-scope stores): up to 8 job counters (one per queue, 128 bytes apart), then the per
// (batch x head, query block) counts of stored dU quadrants, four per (query block, key block) pair.
constexpr int kKvqJob = 0, kKvqJobStride = 32, kKvqCounts = 256;
// Polls of a count before a query job's wait gives up (seconds; no wait of a correct launch comes
// near it): the job then writes its dP1 rows as NaN instead of hanging the GPU.
constexpr int kKvqSpinLimit = 1 << 20;

int device_cu_count();  // compute units of the current device (relation_bwd_tiles.hip)

// The (query block, key block) pairs of 64 x 64 that hold a visible element (key position below the
// query position): query block qb sees key blocks [0, nkb(qb)). Every block but the last holds 64
// queries, so nkb(qb) = qb + A with A = (q_start + 126) / 64 there and the pairs of query block qb
// start at qb (qb - 1) / 2 + A qb.
struct PairTable {
  __host__ __device__ static int nkb(int qb, int TQ, int q_start) {
    const int qlast = (TQ < 64 * qb + 64 ? TQ : 64 * qb + 64) - 1;
    return (q_start + qlast + 63) / 64;  // keys j < q_start + qlast
  }
  __host__ __device__ static int64_t offset(int qb, int q_start) {
    const int64_t A = (q_start + 126) / 64;
    return int64_t(qb) * (qb - 1) / 2 + A * qb;
  }
  __host__ __device__ static int64_t total(int TQ, int q_start) {
    if (TQ <= 0) return 0;
    const int nqb = (TQ + 63) / 64;
    return offset(nqb - 1, q_start) + nkb(nqb - 1, TQ, q_start);
  }
};

// dlam = the fixed-order sum of the n row-block partials (the rows stage writes them), by the NT
// threads of one workgroup through `red` (NT floats of LDS); every thread must call it.
template <int NT = 256>
__device__ __forceinline__ void dlam_sum(const float* part, int n, float* out, float* red) {
  float acc = 0.f;
  for (int i = threadIdx.x; i < n; i += NT) acc += part[i];
  red[threadIdx.x] = acc;
  __syncthreads();
  for (int w = NT / 2; w >= 1; w >>= 1) {
    if ((int)threadIdx.x < w) red[threadIdx.x] += red[threadIdx.x + w];
    __syncthreads();
  }
  if (threadIdx.x == 0) *out = red[0];
}

// bf16 with D in {32, 64, 96, 128}: the atomic-free tile kernels (dP2 / dI~ key-stationary, then dP1
// query-stationary), for the stages selected in `stages` (MOTE_BWD_KEYS, MOTE_BWD_QUERIES).
void launch_bwd_tiles(const BwdParams& p, int stages, hipStream_t stream);

}  // namespace mote
