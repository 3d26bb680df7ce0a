// mote_abi_layout(): the size of every argument struct of include/mote_relation.h and the offset and
// size of each of its fields, as this compiler lays them out, so a binding written by hand (ctypes,
// cgo, JNI) can check its mirror of the structs against the library it loads. Host code only.
#include <stddef.h>

#include <mutex>
#include <string>

#include "mote_relation.h"

namespace {

struct Entry {
  const char* type;
  const char* field;  // "" for the struct's own size
  size_t offset, size;
};

#define MOTE_STRUCT(S) Entry{#S, "", 0, sizeof(S)}
#define F(S, f) Entry{#S, #f, offsetof(S, f), sizeof(((S*)nullptr)->f)}

const Entry kLayout[] = {
    MOTE_STRUCT(mote_view),
    F(mote_view, data), F(mote_view, stride_b), F(mote_view, stride_h), F(mote_view, stride_r),
    MOTE_STRUCT(mote_relation_fwd_args),
    F(mote_relation_fwd_args, dtype), F(mote_relation_fwd_args, B), F(mote_relation_fwd_args, H),
    F(mote_relation_fwd_args, TQ), F(mote_relation_fwd_args, TK), F(mote_relation_fwd_args, D),
    F(mote_relation_fwd_args, q_start), F(mote_relation_fwd_args, tau_s), F(mote_relation_fwd_args, p1),
    F(mote_relation_fwd_args, p2), F(mote_relation_fwd_args, info), F(mote_relation_fwd_args, y),
    F(mote_relation_fwd_args, ibar), F(mote_relation_fwd_args, lse), F(mote_relation_fwd_args, g),
    F(mote_relation_fwd_args, lam), F(mote_relation_fwd_args, cu_seqlens),
    F(mote_relation_fwd_args, total_rows), F(mote_relation_fwd_args, workspace),
    F(mote_relation_fwd_args, workspace_bytes),
    MOTE_STRUCT(mote_relation_bwd_args),
    F(mote_relation_bwd_args, dtype), F(mote_relation_bwd_args, B), F(mote_relation_bwd_args, H),
    F(mote_relation_bwd_args, TQ), F(mote_relation_bwd_args, TK), F(mote_relation_bwd_args, D),
    F(mote_relation_bwd_args, q_start), F(mote_relation_bwd_args, tau_s),
    F(mote_relation_bwd_args, deterministic), F(mote_relation_bwd_args, p1), F(mote_relation_bwd_args, p2),
    F(mote_relation_bwd_args, info), F(mote_relation_bwd_args, dy), F(mote_relation_bwd_args, ibar),
    F(mote_relation_bwd_args, lse), F(mote_relation_bwd_args, g), F(mote_relation_bwd_args, dp1),
    F(mote_relation_bwd_args, dp2), F(mote_relation_bwd_args, dinfo), F(mote_relation_bwd_args, dlam),
    F(mote_relation_bwd_args, workspace), F(mote_relation_bwd_args, workspace_bytes),
    F(mote_relation_bwd_args, stages),
    MOTE_STRUCT(mote_rope_givens_args),
    F(mote_rope_givens_args, dtype), F(mote_rope_givens_args, B), F(mote_rope_givens_args, T),
    F(mote_rope_givens_args, H), F(mote_rope_givens_args, D), F(mote_rope_givens_args, pos0),
    F(mote_rope_givens_args, layer_parity), F(mote_rope_givens_args, inv_freq),
    F(mote_rope_givens_args, theta), F(mote_rope_givens_args, qkv), F(mote_rope_givens_args, qkv_sb),
    F(mote_rope_givens_args, qkv_sr), F(mote_rope_givens_args, p1), F(mote_rope_givens_args, p2),
    F(mote_rope_givens_args, info),
    MOTE_STRUCT(mote_rope_givens_bwd_args),
    F(mote_rope_givens_bwd_args, dtype), F(mote_rope_givens_bwd_args, B), F(mote_rope_givens_bwd_args, T),
    F(mote_rope_givens_bwd_args, H), F(mote_rope_givens_bwd_args, D), F(mote_rope_givens_bwd_args, pos0),
    F(mote_rope_givens_bwd_args, layer_parity), F(mote_rope_givens_bwd_args, inv_freq),
    F(mote_rope_givens_bwd_args, theta), F(mote_rope_givens_bwd_args, qkv),
    F(mote_rope_givens_bwd_args, qkv_sb), F(mote_rope_givens_bwd_args, qkv_sr),
    F(mote_rope_givens_bwd_args, qkv_info_only), F(mote_rope_givens_bwd_args, dp1),
    F(mote_rope_givens_bwd_args, dp2), F(mote_rope_givens_bwd_args, dinfo),
    F(mote_rope_givens_bwd_args, dqkv), F(mote_rope_givens_bwd_args, dqkv_sb),
    F(mote_rope_givens_bwd_args, dqkv_sr), F(mote_rope_givens_bwd_args, dtheta),
    F(mote_rope_givens_bwd_args, workspace), F(mote_rope_givens_bwd_args, workspace_bytes),
    MOTE_STRUCT(mote_relation_decode_args),
    F(mote_relation_decode_args, dtype), F(mote_relation_decode_args, B), F(mote_relation_decode_args, H),
    F(mote_relation_decode_args, D), F(mote_relation_decode_args, capacity),
    F(mote_relation_decode_args, layer_parity), F(mote_relation_decode_args, flags),
    F(mote_relation_decode_args, tau_s), F(mote_relation_decode_args, lam),
    F(mote_relation_decode_args, inv_freq), F(mote_relation_decode_args, theta),
    F(mote_relation_decode_args, S), F(mote_relation_decode_args, p1), F(mote_relation_decode_args, p2),
    F(mote_relation_decode_args, info), F(mote_relation_decode_args, in_sb),
    F(mote_relation_decode_args, cache_p2), F(mote_relation_decode_args, cache_info),
    F(mote_relation_decode_args, y), F(mote_relation_decode_args, y_sb), F(mote_relation_decode_args, g),
    F(mote_relation_decode_args, workspace), F(mote_relation_decode_args, workspace_bytes),
    F(mote_relation_decode_args, xm), F(mote_relation_decode_args, run),
    F(mote_relation_decode_args, static_slot),
    MOTE_STRUCT(mote_add_rms_norm_args),
    F(mote_add_rms_norm_args, dtype), F(mote_add_rms_norm_args, res_dtype),
    F(mote_add_rms_norm_args, out_dtype), F(mote_add_rms_norm_args, res_out_dtype),
    F(mote_add_rms_norm_args, rows), F(mote_add_rms_norm_args, D), F(mote_add_rms_norm_args, eps),
    F(mote_add_rms_norm_args, x), F(mote_add_rms_norm_args, x_sr), F(mote_add_rms_norm_args, residual),
    F(mote_add_rms_norm_args, res_sr), F(mote_add_rms_norm_args, weight), F(mote_add_rms_norm_args, y),
    F(mote_add_rms_norm_args, y_sr), F(mote_add_rms_norm_args, residual_out),
    F(mote_add_rms_norm_args, res_out_sr), F(mote_add_rms_norm_args, rstd),
    MOTE_STRUCT(mote_add_rms_norm_bwd_args),
    F(mote_add_rms_norm_bwd_args, dtype), F(mote_add_rms_norm_bwd_args, dres_out_dtype),
    F(mote_add_rms_norm_bwd_args, s_dtype), F(mote_add_rms_norm_bwd_args, dx_dtype),
    F(mote_add_rms_norm_bwd_args, dres_dtype), F(mote_add_rms_norm_bwd_args, rows),
    F(mote_add_rms_norm_bwd_args, D), F(mote_add_rms_norm_bwd_args, dy), F(mote_add_rms_norm_bwd_args, dy_sr),
    F(mote_add_rms_norm_bwd_args, dres_out), F(mote_add_rms_norm_bwd_args, dres_out_sr),
    F(mote_add_rms_norm_bwd_args, s), F(mote_add_rms_norm_bwd_args, s_sr),
    F(mote_add_rms_norm_bwd_args, rstd), F(mote_add_rms_norm_bwd_args, weight),
    F(mote_add_rms_norm_bwd_args, dx), F(mote_add_rms_norm_bwd_args, dx_sr),
    F(mote_add_rms_norm_bwd_args, dresidual), F(mote_add_rms_norm_bwd_args, dres_sr),
    F(mote_add_rms_norm_bwd_args, dweight), F(mote_add_rms_norm_bwd_args, workspace),
    F(mote_add_rms_norm_bwd_args, workspace_bytes),
    MOTE_STRUCT(mote_qkv_rope_args),
    F(mote_qkv_rope_args, B), F(mote_qkv_rope_args, T), F(mote_qkv_rope_args, H), F(mote_qkv_rope_args, D),
    F(mote_qkv_rope_args, pos0), F(mote_qkv_rope_args, layer_parity), F(mote_qkv_rope_args, x),
    F(mote_qkv_rope_args, x_sb), F(mote_qkv_rope_args, x_sr), F(mote_qkv_rope_args, w),
    F(mote_qkv_rope_args, w_sr), F(mote_qkv_rope_args, inv_freq), F(mote_qkv_rope_args, theta),
    F(mote_qkv_rope_args, p1), F(mote_qkv_rope_args, p2), F(mote_qkv_rope_args, info),
    F(mote_qkv_rope_args, info_raw), F(mote_qkv_rope_args, ir_sb), F(mote_qkv_rope_args, ir_sr),
    F(mote_qkv_rope_args, workspace), F(mote_qkv_rope_args, workspace_bytes),
    F(mote_qkv_rope_args, table_ready), F(mote_qkv_rope_args, norm_w1), F(mote_qkv_rope_args, norm_w2),
    F(mote_qkv_rope_args, norm_eps), F(mote_qkv_rope_args, qk_raw), F(mote_qkv_rope_args, qr_sb),
    F(mote_qkv_rope_args, qr_sr),
    MOTE_STRUCT(mote_head_norm_bwd_args),
    F(mote_head_norm_bwd_args, dtype), F(mote_head_norm_bwd_args, rows), F(mote_head_norm_bwd_args, parts),
    F(mote_head_norm_bwd_args, H), F(mote_head_norm_bwd_args, D), F(mote_head_norm_bwd_args, eps),
    F(mote_head_norm_bwd_args, x), F(mote_head_norm_bwd_args, x_sr), F(mote_head_norm_bwd_args, dy),
    F(mote_head_norm_bwd_args, dy_sr), F(mote_head_norm_bwd_args, dx), F(mote_head_norm_bwd_args, dx_sr),
    F(mote_head_norm_bwd_args, gain0), F(mote_head_norm_bwd_args, gain1), F(mote_head_norm_bwd_args, dgain0),
    F(mote_head_norm_bwd_args, dgain1), F(mote_head_norm_bwd_args, workspace),
    F(mote_head_norm_bwd_args, workspace_bytes),
    MOTE_STRUCT(mote_gate_product_args),
    F(mote_gate_product_args, B), F(mote_gate_product_args, T), F(mote_gate_product_args, D),
    F(mote_gate_product_args, x), F(mote_gate_product_args, x_sr), F(mote_gate_product_args, w),
    F(mote_gate_product_args, w_sr), F(mote_gate_product_args, y), F(mote_gate_product_args, y_sr),
    F(mote_gate_product_args, z), F(mote_gate_product_args, s), F(mote_gate_product_args, z_sr),
    MOTE_STRUCT(mote_skinny_gemm_args),
    F(mote_skinny_gemm_args, dtype), F(mote_skinny_gemm_args, B), F(mote_skinny_gemm_args, N),
    F(mote_skinny_gemm_args, K), F(mote_skinny_gemm_args, x), F(mote_skinny_gemm_args, x_sr),
    F(mote_skinny_gemm_args, w), F(mote_skinny_gemm_args, w_sr), F(mote_skinny_gemm_args, y),
    F(mote_skinny_gemm_args, y_sr), F(mote_skinny_gemm_args, run), F(mote_skinny_gemm_args, g),
    F(mote_skinny_gemm_args, xm), F(mote_skinny_gemm_args, heads),
    MOTE_STRUCT(mote_wgrad_args),
    F(mote_wgrad_args, dtype), F(mote_wgrad_args, M), F(mote_wgrad_args, N), F(mote_wgrad_args, K),
    F(mote_wgrad_args, a), F(mote_wgrad_args, a_sr), F(mote_wgrad_args, x), F(mote_wgrad_args, x_sr),
    F(mote_wgrad_args, dw), F(mote_wgrad_args, dw_sr), F(mote_wgrad_args, workspace),
    F(mote_wgrad_args, workspace_bytes),
    MOTE_STRUCT(mote_page_copy_args),
    F(mote_page_copy_args, to_page), F(mote_page_copy_args, planes), F(mote_page_copy_args, H),
    F(mote_page_copy_args, D), F(mote_page_copy_args, elem_bytes), F(mote_page_copy_args, rows),
    F(mote_page_copy_args, arena), F(mote_page_copy_args, a_plane), F(mote_page_copy_args, a_head),
    F(mote_page_copy_args, arena_row0), F(mote_page_copy_args, page), F(mote_page_copy_args, p_plane),
    F(mote_page_copy_args, p_head), F(mote_page_copy_args, page_row0),
    MOTE_STRUCT(mote_chunk_route_args),
    F(mote_chunk_route_args, B), F(mote_chunk_route_args, L), F(mote_chunk_route_args, mask),
    F(mote_chunk_route_args, mask_sr), F(mote_chunk_route_args, cum), F(mote_chunk_route_args, perm),
    F(mote_chunk_route_args, num), F(mote_chunk_route_args, cu_seqlens),
    MOTE_STRUCT(mote_chunk_gather_args),
    F(mote_chunk_gather_args, dtype), F(mote_chunk_gather_args, B), F(mote_chunk_gather_args, L),
    F(mote_chunk_gather_args, M), F(mote_chunk_gather_args, D), F(mote_chunk_gather_args, hidden),
    F(mote_chunk_gather_args, h_sb), F(mote_chunk_gather_args, h_sr), F(mote_chunk_gather_args, perm),
    F(mote_chunk_gather_args, num), F(mote_chunk_gather_args, cu_seqlens), F(mote_chunk_gather_args, out),
    F(mote_chunk_gather_args, o_sb), F(mote_chunk_gather_args, o_sr),
    MOTE_STRUCT(mote_chunk_gather_bwd_args),
    F(mote_chunk_gather_bwd_args, dtype), F(mote_chunk_gather_bwd_args, B), F(mote_chunk_gather_bwd_args, L),
    F(mote_chunk_gather_bwd_args, M), F(mote_chunk_gather_bwd_args, D), F(mote_chunk_gather_bwd_args, dout),
    F(mote_chunk_gather_bwd_args, g_sb), F(mote_chunk_gather_bwd_args, g_sr),
    F(mote_chunk_gather_bwd_args, mask), F(mote_chunk_gather_bwd_args, mask_sr),
    F(mote_chunk_gather_bwd_args, cum), F(mote_chunk_gather_bwd_args, num),
    F(mote_chunk_gather_bwd_args, cu_seqlens), F(mote_chunk_gather_bwd_args, dhidden),
    F(mote_chunk_gather_bwd_args, dh_sb), F(mote_chunk_gather_bwd_args, dh_sr),
    MOTE_STRUCT(mote_dechunk_args),
    F(mote_dechunk_args, dtype), F(mote_dechunk_args, prob_dtype), F(mote_dechunk_args, out_dtype),
    F(mote_dechunk_args, B), F(mote_dechunk_args, L), F(mote_dechunk_args, M), F(mote_dechunk_args, D),
    F(mote_dechunk_args, eps), F(mote_dechunk_args, hidden), F(mote_dechunk_args, h_sb),
    F(mote_dechunk_args, h_sr), F(mote_dechunk_args, prob), F(mote_dechunk_args, p_sb),
    F(mote_dechunk_args, p_sr), F(mote_dechunk_args, perm), F(mote_dechunk_args, num),
    F(mote_dechunk_args, cum), F(mote_dechunk_args, init), F(mote_dechunk_args, out),
    F(mote_dechunk_args, o_sb), F(mote_dechunk_args, o_sr), F(mote_dechunk_args, w),
    F(mote_dechunk_args, workspace), F(mote_dechunk_args, workspace_bytes),
    MOTE_STRUCT(mote_dechunk_bwd_args),
    F(mote_dechunk_bwd_args, dtype), F(mote_dechunk_bwd_args, prob_dtype),
    F(mote_dechunk_bwd_args, dout_dtype), F(mote_dechunk_bwd_args, dx_dtype),
    F(mote_dechunk_bwd_args, dprob_dtype), F(mote_dechunk_bwd_args, B), F(mote_dechunk_bwd_args, L),
    F(mote_dechunk_bwd_args, M), F(mote_dechunk_bwd_args, D), F(mote_dechunk_bwd_args, eps),
    F(mote_dechunk_bwd_args, dout), F(mote_dechunk_bwd_args, g_sb), F(mote_dechunk_bwd_args, g_sr),
    F(mote_dechunk_bwd_args, hidden), F(mote_dechunk_bwd_args, h_sb), F(mote_dechunk_bwd_args, h_sr),
    F(mote_dechunk_bwd_args, prob), F(mote_dechunk_bwd_args, p_sb), F(mote_dechunk_bwd_args, p_sr),
    F(mote_dechunk_bwd_args, perm), F(mote_dechunk_bwd_args, num), F(mote_dechunk_bwd_args, mask),
    F(mote_dechunk_bwd_args, mask_sr), F(mote_dechunk_bwd_args, cum), F(mote_dechunk_bwd_args, w),
    F(mote_dechunk_bwd_args, dhidden), F(mote_dechunk_bwd_args, dh_sb), F(mote_dechunk_bwd_args, dh_sr),
    F(mote_dechunk_bwd_args, dprob), F(mote_dechunk_bwd_args, dp_sb), F(mote_dechunk_bwd_args, dp_sr),
    F(mote_dechunk_bwd_args, workspace), F(mote_dechunk_bwd_args, workspace_bytes),
    MOTE_STRUCT(mote_dechunk_step_args),
    F(mote_dechunk_step_args, prob_dtype), F(mote_dechunk_step_args, hidden_dtype),
    F(mote_dechunk_step_args, state_dtype), F(mote_dechunk_step_args, B), F(mote_dechunk_step_args, D),
    F(mote_dechunk_step_args, eps), F(mote_dechunk_step_args, mask), F(mote_dechunk_step_args, prob),
    F(mote_dechunk_step_args, p_sr), F(mote_dechunk_step_args, hidden), F(mote_dechunk_step_args, h_sr),
    F(mote_dechunk_step_args, last_value), F(mote_dechunk_step_args, l_sr), F(mote_dechunk_step_args, out),
    F(mote_dechunk_step_args, o_sr),
};

#undef F
#undef MOTE_STRUCT

}  // namespace

extern "C" const char* mote_abi_layout(void) {
  // "type size;field offset size;..." with one line per struct, built once
  static std::once_flag once;
  static std::string text;
  std::call_once(once, [] {
    for (const Entry& e : kLayout) {
      if (e.field[0] == 0) {
        if (!text.empty()) text += "\n";
        text += std::string(e.type) + " " + std::to_string(e.size);
      } else {
        text += ";" + std::string(e.field) + " " + std::to_string(e.offset) + " " + std::to_string(e.size);
      }
    }
  });
  return text.c_str();
}
