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
  int B, H, TQ, TK, D, q_start, TQp;
  float scale, tau_inv;
};

constexpr int kRowBlock = 64;  // rows per workgroup in the rows stage; also TQp's granularity

// bf16 with D in {32, 64, 96, 128}: the atomic-free tile kernels (dP2 / dI~ key-stationary, then dP1
// query-stationary), for the stages selected in `stages` (MOTE_BWD_KEYS, MOTE_BWD_QUERIES).
void launch_bwd_tiles(const BwdParams& p, int stages, hipStream_t stream);

}  // namespace mote
