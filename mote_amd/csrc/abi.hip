// extern "C" entry points of libmote_relation.so (declared in include/mote_relation.h).
//
// The entry points validate their arguments, translate the argument blocks into kernel parameter
// blocks and launch on the caller's stream. They allocate nothing and never synchronise; the only
// mutable state is the thread-local error text.
#include <stdarg.h>
#include <stdio.h>

#include "params.hpp"

namespace mote {

static thread_local char g_err[512] = "";

int set_error(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof(g_err), fmt, ap);
  va_end(ap);
  return code;
}

int check_launch(const char* what) {
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) return set_error(MOTE_ERR_LAUNCH, "%s: launch failed: %s", what, hipGetErrorString(e));
  return MOTE_OK;
}

// wgrad.hip (kept out of params.hpp, whose text every recorded kernel profile is tied to)
size_t wgrad_workspace_bytes(const mote_wgrad_args* a);
int launch_wgrad(const mote_wgrad_args* a, hipStream_t stream);

}  // namespace mote

extern "C" {

const char* mote_last_error(void) { return mote::g_err; }

const char* mote_version(void) { return "mote_relation 0.1 gfx950"; }

size_t mote_relation_fwd_workspace(const mote_relation_fwd_args* args) {
  return args ? mote::fwd_workspace_bytes(args) : 0;
}

int mote_relation_fwd(const mote_relation_fwd_args* args, void* stream) {
  mote::g_err[0] = 0;
  return mote::launch_fwd(args, reinterpret_cast<hipStream_t>(stream));
}

size_t mote_relation_bwd_workspace(const mote_relation_bwd_args* args) {
  return args ? mote::bwd_workspace_bytes(args) : 0;
}

int mote_relation_bwd(const mote_relation_bwd_args* args, void* stream) {
  mote::g_err[0] = 0;
  return mote::launch_bwd(args, reinterpret_cast<hipStream_t>(stream));
}

int mote_rope_givens_fwd(const mote_rope_givens_args* args, void* stream) {
  mote::g_err[0] = 0;
  return mote::launch_rope_givens_fwd(args, reinterpret_cast<hipStream_t>(stream));
}

size_t mote_rope_givens_bwd_workspace(const mote_rope_givens_bwd_args* args) {
  return args ? mote::rope_givens_bwd_workspace_bytes(args) : 0;
}

int mote_rope_givens_bwd(const mote_rope_givens_bwd_args* args, void* stream) {
  mote::g_err[0] = 0;
  return mote::launch_rope_givens_bwd(args, reinterpret_cast<hipStream_t>(stream));
}

size_t mote_relation_decode_workspace(const mote_relation_decode_args* args) {
  return args ? mote::decode_workspace_bytes(args) : 0;
}

int mote_relation_decode(const mote_relation_decode_args* args, void* stream) {
  mote::g_err[0] = 0;
  return mote::launch_decode(args, reinterpret_cast<hipStream_t>(stream));
}

int mote_relation_decode_static(const mote_relation_decode_args* args, void* stream) {
  mote::g_err[0] = 0;
  return mote::launch_decode_static(args, reinterpret_cast<hipStream_t>(stream));
}

int mote_add_rms_norm_fwd(const mote_add_rms_norm_args* args, void* stream) {
  mote::g_err[0] = 0;
  return mote::launch_add_rms_norm_fwd(args, reinterpret_cast<hipStream_t>(stream));
}

size_t mote_add_rms_norm_bwd_workspace(const mote_add_rms_norm_bwd_args* args) {
  return args ? mote::add_rms_norm_bwd_workspace_bytes(args) : 0;
}

int mote_add_rms_norm_bwd(const mote_add_rms_norm_bwd_args* args, void* stream) {
  mote::g_err[0] = 0;
  return mote::launch_add_rms_norm_bwd(args, reinterpret_cast<hipStream_t>(stream));
}

size_t mote_qkv_rope_workspace(const mote_qkv_rope_args* args) {
  return args ? mote::qkv_rope_workspace_bytes(args) : 0;
}

int mote_qkv_rope_fwd(const mote_qkv_rope_args* args, void* stream) {
  mote::g_err[0] = 0;
  return mote::launch_qkv_rope_fwd(args, reinterpret_cast<hipStream_t>(stream));
}

int mote_gate_product(const mote_gate_product_args* args, void* stream) {
  mote::g_err[0] = 0;
  return mote::launch_gate_product(args, reinterpret_cast<hipStream_t>(stream));
}

int mote_arena_page_copy(const mote_page_copy_args* args, void* stream) {
  mote::g_err[0] = 0;
  return mote::launch_page_copy(args, reinterpret_cast<hipStream_t>(stream));
}

int mote_skinny_gemm(const mote_skinny_gemm_args* args, void* stream) {
  mote::g_err[0] = 0;
  return mote::launch_skinny_gemm(args, reinterpret_cast<hipStream_t>(stream));
}

size_t mote_wgrad_workspace(const mote_wgrad_args* args) { return args ? mote::wgrad_workspace_bytes(args) : 0; }

int mote_wgrad(const mote_wgrad_args* args, void* stream) {
  mote::g_err[0] = 0;
  return mote::launch_wgrad(args, reinterpret_cast<hipStream_t>(stream));
}

int mote_chunk_route(const mote_chunk_route_args* args, void* stream) {
  mote::g_err[0] = 0;
  return mote::launch_chunk_route(args, reinterpret_cast<hipStream_t>(stream));
}

int mote_chunk_gather(const mote_chunk_gather_args* args, void* stream) {
  mote::g_err[0] = 0;
  return mote::launch_chunk_gather(args, reinterpret_cast<hipStream_t>(stream));
}

int mote_chunk_gather_bwd(const mote_chunk_gather_bwd_args* args, void* stream) {
  mote::g_err[0] = 0;
  return mote::launch_chunk_gather_bwd(args, reinterpret_cast<hipStream_t>(stream));
}

size_t mote_dechunk_workspace(const mote_dechunk_args* args) {
  return args ? mote::dechunk_workspace_bytes(args) : 0;
}

int mote_dechunk_fwd(const mote_dechunk_args* args, void* stream) {
  mote::g_err[0] = 0;
  return mote::launch_dechunk_fwd(args, reinterpret_cast<hipStream_t>(stream));
}

size_t mote_dechunk_bwd_workspace(const mote_dechunk_bwd_args* args) {
  return args ? mote::dechunk_bwd_workspace_bytes(args) : 0;
}

int mote_dechunk_bwd(const mote_dechunk_bwd_args* args, void* stream) {
  mote::g_err[0] = 0;
  return mote::launch_dechunk_bwd(args, reinterpret_cast<hipStream_t>(stream));
}

int mote_dechunk_step(const mote_dechunk_step_args* args, void* stream) {
  mote::g_err[0] = 0;
  return mote::launch_dechunk_step(args, reinterpret_cast<hipStream_t>(stream));
}

}  // extern "C"
