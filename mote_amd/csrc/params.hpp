// Kernel parameter blocks (device side) and launcher declarations shared by the .hip files.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/mote_relation.h"

namespace mote {

// Forward: dense [B,H,T,D] batches or cu_seqlens-packed sequences (see mote_relation_fwd_args).
struct FwdParams {
  const void* p1;
  const void* p2;
  const void* info;
  void* y;
  float* ibar;
  float* lse;
  float* g;
  const float* lam;
  const int32_t* cu;  // null in dense mode
  float* part;        // split partials [nseq][H][nqb][2][64 * DP + 128] (null: no split)
  int split_c;        // query blocks with more key blocks than this run as two halves
  int* jobs;          // persistent tile launch: one job counter per queue, 32 ints apart (null: one job per workgroup)
  int jobs_nq;        // its queue count (heads h go to queue h % jobs_nq)
  int64_t q_sb, q_sh, q_sr;
  int64_t k_sb, k_sh, k_sr;
  int64_t v_sb, v_sh, v_sr;
  int64_t y_sb, y_sh, y_sr;
  int nseq, H, TQ, TK, D, q_start, total_rows, nqb;
  float scale, tau_inv;
};

int launch_fwd(const mote_relation_fwd_args* a, hipStream_t stream);
size_t fwd_workspace_bytes(const mote_relation_fwd_args* a);
int launch_bwd(const mote_relation_bwd_args* a, hipStream_t stream);
size_t bwd_workspace_bytes(const mote_relation_bwd_args* a);
int launch_rope_givens_fwd(const mote_rope_givens_args* a, hipStream_t stream);
int launch_rope_givens_bwd(const mote_rope_givens_bwd_args* a, hipStream_t stream);
size_t rope_givens_bwd_workspace_bytes(const mote_rope_givens_bwd_args* a);
int launch_decode(const mote_relation_decode_args* a, hipStream_t stream);
int launch_decode_static(const mote_relation_decode_args* a, hipStream_t stream);
size_t decode_workspace_bytes(const mote_relation_decode_args* a);
int launch_add_rms_norm_fwd(const mote_add_rms_norm_args* a, hipStream_t stream);
int launch_add_rms_norm_bwd(const mote_add_rms_norm_bwd_args* a, hipStream_t stream);
size_t add_rms_norm_bwd_workspace_bytes(const mote_add_rms_norm_bwd_args* a);
int launch_chunk_route(const mote_chunk_route_args* a, hipStream_t stream);
size_t qkv_rope_workspace_bytes(const mote_qkv_rope_args* a);
int launch_qkv_rope_fwd(const mote_qkv_rope_args* a, hipStream_t stream);
int launch_gate_product(const mote_gate_product_args* a, hipStream_t stream);
int launch_page_copy(const mote_page_copy_args* a, hipStream_t stream);
int launch_skinny_gemm(const mote_skinny_gemm_args* a, hipStream_t stream);
int launch_chunk_gather(const mote_chunk_gather_args* a, hipStream_t stream);
int launch_chunk_gather_bwd(const mote_chunk_gather_bwd_args* a, hipStream_t stream);
size_t dechunk_workspace_bytes(const mote_dechunk_args* a);
int launch_dechunk_fwd(const mote_dechunk_args* a, hipStream_t stream);
size_t dechunk_bwd_workspace_bytes(const mote_dechunk_bwd_args* a);
int launch_dechunk_bwd(const mote_dechunk_bwd_args* a, hipStream_t stream);
int launch_dechunk_step(const mote_dechunk_step_args* a, hipStream_t stream);

// Error reporting shared by the launchers (thread-local text, see abi.cpp).
int set_error(int code, const char* fmt, ...);
int check_launch(const char* what);

// The tile kernels address staged rows with 32-bit offsets from the block's first row.
inline bool tile_strides_ok(const mote_view& a, const mote_view& b, const mote_view& c) {
  const int64_t lim = int64_t(1) << 24;
  return a.stride_r >= 0 && a.stride_r < lim && b.stride_r >= 0 && b.stride_r < lim && c.stride_r >= 0 &&
         c.stride_r < lim;
}

// The padded head dim a kernel instance is compiled for: D rounded up to 32 (D <= 128, D % 8 == 0).
inline int padded_dim(int D) { return D <= 32 ? 32 : D <= 64 ? 64 : D <= 96 ? 96 : 128; }

}  // namespace mote
