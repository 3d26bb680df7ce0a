/* mote_relation.h — C ABI of the MI355X (gfx950) Relation library, libmote_relation.so.
 *
 * The library holds the hand-written HIP kernels of Mote's Relation mixer. Every entry point takes
 * plain device pointers, sizes and element strides, launches on the caller's HIP stream and
 * returns a status code; it allocates nothing, keeps no reference to its arguments after it
 * returns and never synchronises the device. `mote_last_error()` explains a non-zero status.
 * Entry points are reentrant: the only mutable state is the thread-local error text.
 *
 * Reference interfaces (noahsabaj/mote, paths relative to its source root) are cited per function.
 */
#ifndef MOTE_RELATION_H
#define MOTE_RELATION_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Status codes. */
enum {
  MOTE_OK = 0,
  MOTE_ERR_ARGUMENT = 1,    /* null pointer, bad enum, inconsistent sizes */
  MOTE_ERR_SHAPE = 2,       /* shape outside what the kernels support (e.g. D > 128, D % 8 != 0) */
  MOTE_ERR_WORKSPACE = 3,   /* workspace smaller than the matching *_workspace() query */
  MOTE_ERR_LAUNCH = 4       /* the HIP runtime refused a launch */
};

/* Element types of the input/output tensors. Statistics are always fp32. */
enum { MOTE_F32 = 0, MOTE_BF16 = 1 };

/* A [batch, heads, rows, D] tensor view with unit stride along D; strides count elements. */
typedef struct mote_view {
  void* data;
  int64_t stride_b;
  int64_t stride_h;
  int64_t stride_r;
} mote_view;

/* Text of the last error on this thread ("" when none). */
const char* mote_last_error(void);

/* Library version and the GPU architecture its kernels were built for ("gfx950"). */
const char* mote_version(void);

/* The layout of every argument struct below as this library was compiled: one line per struct,
 * "name size;field offset size;..." (bytes, fields in declaration order), so a binding that mirrors
 * the structs by hand (ctypes, cgo, JNI) can check itself against the library it loads. No
 * counterpart in the reference, whose kernels take Python arguments. */
const char* mote_abi_layout(void);

/* Measurement helper, no counterpart in the reference: the shader clock at the moment of the call.
 * One launch of `workgroups` workgroups (256 threads) that each run `iters` steps of matrix-core
 * products and exponentials; out (device, int64, 3 per workgroup) receives workgroup i's count of
 * the shader clock (s_memtime) over its loop, the count of the constant 100 MHz clock
 * (s_memrealtime) over the same span, and a value that keeps the work alive. Shader clock in MHz =
 * 100 * out[3 i] / out[3 i + 1]. */
int mote_clock_probe(int64_t* out, int workgroups, int iters, void* stream);

/* ------------------------------------------------------------------------------------------------
 * Fused Relation forward.
 * Replaces: the Triton `_fwd_kernel` and its launcher `_launch_fwd`
 * (mote/model/flash_relation.py:76-183, 507-541), behind the custom op `mote::relation_fwd`
 * (flash_relation.py:620-622). Same outputs: y (dtype of info), ibar fp32, lse fp32 (natural
 * units, -inf for rows without a past), g fp32.
 *
 * Dense mode (cu_seqlens == NULL): p1/y are [B, H, TQ, D]; p2/info are [B, H, TK, D] with
 * TK == q_start + TQ (flash_relation.py:511); ibar is [B, H, TQ, D] and lse/g are [B, H, TQ],
 * all contiguous. Any row/head/batch strides are accepted for p1, p2, info and y (the decode
 * arena's head stride capacity*D included, flash_relation.py:513-525).
 * Varlen mode (cu_seqlens != NULL, no counterpart in the reference, which pads instead,
 * mote/model/dc.py:192-218): B sequences packed along the row axis, sequence b owning rows
 * [cu_seqlens[b], cu_seqlens[b+1]); q_start must be 0, TQ = TK = the longest sequence, total_rows =
 * cu_seqlens[B]; stride_b is ignored; ibar is [H, total_rows, D], lse/g are [H, total_rows].
 * Workspace (optional): with at least mote_relation_fwd_workspace() bytes of device memory the
 * longest query blocks are split over two workgroups whose partial softmax states merge in a
 * second launch, which evens out the causal imbalance (rows beyond 96 key blocks), or, with many
 * more query blocks than workgroup slots (B H ceil(TQ / 64) >= 8 per CU), persistent workgroups take
 * the query blocks from job counters held there (cleared by a small launch first); with workspace ==
 * NULL every query block runs in one workgroup. Results are identical up to float rounding of the
 * merge (bit for bit with the persistent workgroups); contents of the workspace on entry do not
 * matter. Calls that share a workspace must not overlap.
 * ------------------------------------------------------------------------------------------------ */
typedef struct mote_relation_fwd_args {
  int dtype;          /* MOTE_F32 or MOTE_BF16, for p1, p2, info and y */
  int B, H, TQ, TK, D, q_start;
  float tau_s;        /* Self temperature (RelationCfg.tau_s, mote/config.py:38) */
  mote_view p1, p2, info, y;
  float* ibar;
  float* lse;
  float* g;
  const float* lam;   /* device pointer to the fp32 count-calibration scalar */
  const int32_t* cu_seqlens;
  int total_rows;
  void* workspace;
  size_t workspace_bytes;
} mote_relation_fwd_args;

size_t mote_relation_fwd_workspace(const mote_relation_fwd_args* args);
int mote_relation_fwd(const mote_relation_fwd_args* args, void* stream);

/* ------------------------------------------------------------------------------------------------
 * Fused Relation backward.
 * Replaces: `_bwd_rows_kernel` + `_bwd_kernel` (one pass, fp32 atomics for dp1) and the
 * deterministic two-pass `_bwd_kv_kernel` + `_bwd_q_kernel` with their launchers
 * (mote/model/flash_relation.py:186-460, 544-615), behind `mote::relation_bwd` (:634-637).
 * Inputs are the forward's inputs and saved statistics (ibar, lse, g as produced by
 * mote_relation_fwd, dense layout) and dy ([B, H, TQ, D], any strides). Outputs dp1 [B,H,TQ,D],
 * dp2 and dinfo [B,H,TK,D] in `dtype` (any strides) and dlam (one fp32, overwritten).
 * bf16 with D in {32, 64, 96, 128} runs atomic-free kernels (key-stationary dp2/dinfo, then
 * query-stationary dp1): every result is bitwise reproducible whatever `deterministic` says.
 * Other shapes (fp32, padded head dims): `deterministic` != 0 selects the atomic-free pair of
 * kernels (the reference's MOTE_DETERMINISTIC_RELATION, flash_relation.py:51), 0 the one-pass
 * kernel with fp32 atomics for dp1.
 * The workspace is caller-allocated device memory of at least mote_relation_bwd_workspace()
 * bytes; its contents on entry do not matter.
 * `stages` selects which launches run (MOTE_BWD_ROWS: per-row terms and operand copies;
 * MOTE_BWD_KEYS: the key-stationary kernel; MOTE_BWD_QUERIES: the query-stationary dp1 kernel,
 * where the path has one; MOTE_BWD_FINISH: dp1 cast and dlam, which the bf16 tile path computes in
 * its MOTE_BWD_QUERIES launch instead); 0 runs all of them. A caller that
 * splits them (to time or overlap them) issues them in that order on one stream with one workspace.
 * On the bf16 tile path with D <= 96, MOTE_BWD_KEYS and MOTE_BWD_QUERIES in one call run as one
 * launch (dp1 bit-identical to the separate launches, dp2 / dinfo the same terms added in another
 * order); the environment variable MOTE_BWD_FUSED=0, read on every call, keeps them separate.
 * ------------------------------------------------------------------------------------------------ */
#define MOTE_BWD_ROWS 1
#define MOTE_BWD_KEYS 2
#define MOTE_BWD_FINISH 4
#define MOTE_BWD_QUERIES 8

typedef struct mote_relation_bwd_args {
  int dtype;
  int B, H, TQ, TK, D, q_start;
  float tau_s;
  int deterministic;
  mote_view p1, p2, info, dy;
  const float* ibar;
  const float* lse;
  const float* g;
  mote_view dp1, dp2, dinfo;
  float* dlam;
  void* workspace;
  size_t workspace_bytes;
  int stages;
} mote_relation_bwd_args;

size_t mote_relation_bwd_workspace(const mote_relation_bwd_args* args);
int mote_relation_bwd(const mote_relation_bwd_args* args, void* stream);

/* ------------------------------------------------------------------------------------------------
 * RoPE on p1/p2 and Givens head mixing on I~, fused with the split of the projection output.
 * Replaces: `_rope_cos_sin` / `rope_tables` / `_apply_rope` and `FullRelation._givens`
 * (mote/model/relation.py:37-68, 160-174) as called from FullRelation.forward (:204-215).
 * qkv is the [B, T, 3*H*D] output of the fused projection [w1; w2; wi] (row stride qkv_sr, batch
 * stride qkv_sb, elements); positions are pos0 .. pos0+T-1. inv_freq is the fp32 [D/2] table
 * 1/theta^(2k/D) (relation.py:39), or NULL for no RoPE (NoPE Relation, relation.py:141).
 * theta is the fp32 [H/2] Givens angle vector, or NULL for no Givens; layer_parity picks the
 * pairing (0: (0,1),(2,3)...; 1: (1,2),...,(H-1,0), relation.py:150-157). The cos/sin factors are
 * rounded to `dtype` before use, as the reference casts them (relation.py:42, 165-166).
 * ------------------------------------------------------------------------------------------------ */
typedef struct mote_rope_givens_args {
  int dtype;
  int B, T, H, D, pos0, layer_parity;
  const float* inv_freq;
  const float* theta;
  const void* qkv;
  int64_t qkv_sb, qkv_sr;
  mote_view p1, p2, info;   /* outputs, [B, H, T, D] views */
} mote_rope_givens_args;

int mote_rope_givens_fwd(const mote_rope_givens_args* args, void* stream);

/* Backward of mote_rope_givens_fwd: gradients dp1, dp2, dinfo ([B,H,T,D] views) -> dqkv
 * ([B, T, 3*H*D], strides dqkv_sb/dqkv_sr) and dtheta (fp32 [H/2], overwritten; deterministic).
 * qkv is the forward's input (needed for dtheta). Workspace: mote_rope_givens_bwd_workspace(). */
typedef struct mote_rope_givens_bwd_args {
  int dtype;
  int B, T, H, D, pos0, layer_parity;
  const float* inv_freq;
  const float* theta;
  const void* qkv;       /* only its I~ columns are read (for d theta) */
  int64_t qkv_sb, qkv_sr;
  int qkv_info_only;     /* 1: qkv holds the I~ projections alone ([B, T, H*D], e.g. mote_qkv_rope_fwd's info_raw) */
  mote_view dp1, dp2, dinfo;
  void* dqkv;
  int64_t dqkv_sb, dqkv_sr;
  float* dtheta;
  void* workspace;
  size_t workspace_bytes;
} mote_rope_givens_bwd_args;

size_t mote_rope_givens_bwd_workspace(const mote_rope_givens_bwd_args* args);
int mote_rope_givens_bwd(const mote_rope_givens_bwd_args* args, void* stream);

/* ------------------------------------------------------------------------------------------------
 * One decode step of one Relation layer over the {P2, I~} cache.
 * Replaces: GraphDecoder._relation_step between the projections and `_out`
 * (mote/infer/graph.py:158-186): RoPE at the device position S, Givens, the cast to the cache
 * dtype, the append of the new P2 / I~ row at S (index_copy_, :173-175), and the masked
 * softmax read of rows [0, S] (:177-185), for B independent sequences (the reference decodes
 * B = 1; B > 1 is B independent batch-1 steps). S[b] (int64, device) is read on the device, so the
 * launch is capturable in a HIP graph with a fixed argument set (graph.py:1-17).
 * Inputs p1/p2/info are the raw projections of the new chunk, [B, H, D] with batch stride in_sb
 * and head stride D, in `dtype` (the cache dtype). Outputs: y [B, H, D] (dtype, batch stride y_sb)
 * and g [B, H] fp32, the exchange mass g = 1 - F_SS (graph.py:186 averages it over heads).
 * The caches are [B, H, capacity, D] views (mote/model/arena.py:30-51, 141-143); rows past S are
 * never read. S[b] >= capacity writes NaN into y[b] and skips the append.
 * flags bit 0 (MOTE_DECODE_ADVANCE): add 1 to every S[b] once the step has read it (graph.py's
 * S += 1, :189-190), so a captured step needs no separate kernel for it.
 * flags bit 1 (MOTE_DECODE_ROPE_F32): RoPE with fp32 cos / sin and fp32 arithmetic, the rotated p1 /
 * p2 rounded once into `dtype`: the graph decoder's convention when its input x is fp32 under serving
 * autocast (graph.py:158-164 builds the tables at x.dtype, :171-172 casts into the arena). Without it
 * the tables are rounded to `dtype` and every product and sum of the rotation is rounded to `dtype`
 * (x in the cache dtype, relation.py:211-214). Givens is in `dtype` either way (relation.py:165-166).
 * One launch on `stream`: a split-S sweep whose last workgroup per (sequence, head) merges the
 * partials. The workspace (mote_relation_decode_workspace() bytes) holds the per-split partials and
 * completion counters: zero-fill it once before its first call (every call leaves the counters at
 * zero again). Calls that share a workspace must not overlap.
 * ------------------------------------------------------------------------------------------------ */
#define MOTE_DECODE_ADVANCE 1
#define MOTE_DECODE_ROPE_F32 2

typedef struct mote_relation_decode_args {
  int dtype;
  int B, H, D, capacity, layer_parity, flags;
  float tau_s;
  const float* lam;
  const float* inv_freq;   /* [D/2] fp32 or NULL (no RoPE) */
  const float* theta;      /* [H/2] fp32 or NULL (no Givens) */
  int64_t* S;              /* [B] positions on the device */
  const void* p1;
  const void* p2;
  const void* info;
  int64_t in_sb;
  mote_view cache_p2, cache_info;
  void* y;
  int64_t y_sb;
  float* g;
  void* workspace;
  size_t workspace_bytes;
  float* xm;               /* [B] mean over the heads of g (graph.py:186), or NULL */
  /* Predicate, or NULL (always run): a device byte (a bool tensor, e.g. the router's boundary bit)
     read by every workgroup; 0 makes the launch write nothing (no append, no advance, no outputs).
     It stands in for the graph decoder's conditional node around the main step (graph.py:44-57,
     224-226): one captured graph serves both branches. */
  const unsigned char* run;
  /* Read by mote_relation_decode_static only (ignored by mote_relation_decode): which of its
     MOTE_DECODE_STATIC_SLOTS scratch copies the call uses, 0 when the block is zero-initialised. */
  int static_slot;
} mote_relation_decode_args;

size_t mote_relation_decode_workspace(const mote_relation_decode_args* args);
int mote_relation_decode(const mote_relation_decode_args* args, void* stream);

/* ------------------------------------------------------------------------------------------------
 * The decode step without a workspace. No counterpart in the reference: it is for callers that
 * cannot allocate device memory (code under HIP graph capture, tight serving loops, harnesses that
 * forbid hipMalloc). Arguments and results are those of mote_relation_decode, whose `workspace` /
 * `workspace_bytes` fields are ignored: the per-split partials and completion counters live in a
 * static device array of MOTE_DECODE_STATIC_SLOTS slots of MOTE_DECODE_STATIC_BYTES bytes each per
 * GPU, held until the process ends; `static_slot` picks the slot (anything outside
 * [0, MOTE_DECODE_STATIC_SLOTS) is refused with MOTE_ERR_ARGUMENT). A call takes at most 256
 * sequences and 1024 sequence-heads (B * H); anything beyond is refused with MOTE_ERR_WORKSPACE
 * before any launch. Calls on one GPU that use one slot share it: calls ordered on one stream are
 * fine, calls on unordered streams race. Calls on different slots are independent, so a process
 * that decodes on two streams at once (the reference's daemon serves on a stream of its own beside
 * the trainer's, mote/infer/engine.py:150-162) gives each stream a slot of its own.
 * The first call on a slot of a device clears that slot in the caller's stream order and is refused
 * under graph capture (the clear would be captured and rerun on every replay): make it once outside.
 * The stream's device must be the current device. It allocates nothing.
 * ------------------------------------------------------------------------------------------------ */
#define MOTE_DECODE_STATIC_BYTES (1u << 20)
#define MOTE_DECODE_STATIC_SLOTS 4

int mote_relation_decode_static(const mote_relation_decode_args* args, void* stream);

/* ------------------------------------------------------------------------------------------------
 * Fused residual add + RMSNorm (the pre-norm of every H-Net block and the final norm).
 * Replaces: RMSNorm.forward(x, residual, prenorm, residual_in_fp32) (mote/model/norm.py:36-59), whose
 * CUDA path calls mamba_ssm's Triton rms_norm_fn with the same semantics (norm.py:17-23, 48-50).
 * Per row of D elements, in fp32: s = x + residual (residual == NULL: s = x), r = 1/sqrt(mean(s^2) +
 * eps), y = s r weight. x, residual, y and residual_out are [rows, D] with unit element stride and a
 * row stride each (elements); every dtype is MOTE_F32 or MOTE_BF16 independently (residual_in_fp32:
 * residual and residual_out MOTE_F32). The sum is held in res_out_dtype: MOTE_BF16 rounds it before
 * the norm, as `x + residual` in bf16 does (norm.py:51). residual_out (the new residual stream s) and
 * rstd (r, fp32 [rows], kept for the backward) may be NULL. weight is fp32 [D]. Rows must start on
 * 8-byte (bf16) / 16-byte (fp32) boundaries; 4 <= D <= 2048, D % 4 == 0. rows == 0 launches nothing
 * (the data pointers may then be NULL); the backward then only sets dweight to 0.
 * ------------------------------------------------------------------------------------------------ */
typedef struct mote_add_rms_norm_args {
  int dtype;            /* x */
  int res_dtype;        /* residual */
  int out_dtype;        /* y */
  int res_out_dtype;    /* residual_out */
  int rows, D;
  float eps;
  const void* x; int64_t x_sr;
  const void* residual; int64_t res_sr;
  const float* weight;
  void* y; int64_t y_sr;
  void* residual_out; int64_t res_out_sr;
  float* rstd;
} mote_add_rms_norm_args;

int mote_add_rms_norm_fwd(const mote_add_rms_norm_args* args, void* stream);

/* Backward of mote_add_rms_norm_fwd. With g = dy weight and the saved s (residual_out) and r (rstd):
 * ds = r g - (r^3 / D) s sum(g s) + dres_out; dx = ds, dresidual = ds (NULL: no residual input),
 * dweight = sum over rows of dy s r (fp32 [D], overwritten, fixed-order sum: reproducible).
 * dres_out (the gradient reaching the returned residual stream) may be NULL. Workspace:
 * mote_add_rms_norm_bwd_workspace() bytes of device memory, contents on entry do not matter. */
typedef struct mote_add_rms_norm_bwd_args {
  int dtype;            /* dy */
  int dres_out_dtype;
  int s_dtype;
  int dx_dtype;
  int dres_dtype;
  int rows, D;
  const void* dy; int64_t dy_sr;
  const void* dres_out; int64_t dres_out_sr;
  const void* s; int64_t s_sr;
  const float* rstd;
  const float* weight;
  void* dx; int64_t dx_sr;
  void* dresidual; int64_t dres_sr;
  float* dweight;
  void* workspace;
  size_t workspace_bytes;
} mote_add_rms_norm_bwd_args;

size_t mote_add_rms_norm_bwd_workspace(const mote_add_rms_norm_bwd_args* args);
int mote_add_rms_norm_bwd(const mote_add_rms_norm_bwd_args* args, void* stream);

/* ------------------------------------------------------------------------------------------------
 * Fused projection prologue (bf16): qkv = x [w1; w2; wi]^T, RoPE on p1 / p2 and the Givens rotation
 * on I~ in the product's epilogue, written into the three [B, H, T, D] head views; the same results as
 * the projection (x [w1; w2; wi]^T rounded to bf16) followed by mote_rope_givens_fwd.
 * Replaces: the three projections, the optional QK-Norm and the RoPE / Givens of
 * FullRelation.forward (mote/model/relation.py:199-215); the unfused path stays for fp32 and other
 * head dims.
 * x: [B, T, H*D] bf16 with the batches back to back (x_sb == T x_sr); w: [3 H D, H D] bf16 rows
 * w1 | w2 | wi (row stride w_sr); D in {64, 96, 128}; H even; H D % 32 == 0. inv_freq NULL: no RoPE;
 * theta NULL: no Givens. info_raw (may be NULL) receives the I~ projections before the rotation,
 * for mote_rope_givens_bwd (qkv_info_only = 1). Workspace: mote_qkv_rope_workspace() bytes (the
 * cos / sin table of the T positions). table_ready = 1: the workspace already holds that table,
 * written by an earlier call with the same T, pos0 and inv_freq whose work precedes this one on the
 * stream (the caller memoises tables the way the reference memoises its RoPE tables,
 * relation.py:45-58); the table launch is skipped. All rows on 16-byte boundaries.
 * ------------------------------------------------------------------------------------------------ */
typedef struct mote_qkv_rope_args {
  int B, T, H, D;
  int pos0, layer_parity;
  const void* x; int64_t x_sb, x_sr;
  const void* w; int64_t w_sr;
  const float* inv_freq;
  const float* theta;
  mote_view p1, p2, info;
  void* info_raw; int64_t ir_sb, ir_sr;
  void* workspace;
  size_t workspace_bytes;
  int table_ready;
  /* QK-Norm (relation.py:71-94, 208-210), applied to p1 / p2 before RoPE when both gains are given:
     per token and head y = x rsqrt(mean(x^2) + eps) * gain (fp32 gains [D]), rounded to bf16.
     qk_raw (may be NULL; only with the gains) receives the p1 | p2 projections before the norm,
     [B, T, 2 H D] with batch / row strides qr_sb / qr_sr, for the backward. */
  const float* norm_w1;
  const float* norm_w2;
  float norm_eps;
  void* qk_raw; int64_t qr_sb, qr_sr;
} mote_qkv_rope_args;

size_t mote_qkv_rope_workspace(const mote_qkv_rope_args* args);
int mote_qkv_rope_fwd(const mote_qkv_rope_args* args, void* stream);

/* ------------------------------------------------------------------------------------------------
 * Backward of QK-Norm for the fused prologue (bf16).
 * Replaces: the autograd of HeadRMSNorm (mote/model/relation.py:71-94) applied to p1 / p2
 * (:208-210), i.e. the two norms' backward in the prologue's backward. Per token row and head of
 * part p (p1 = part 0, p2 = part 1; part p holds columns [p H D, (p + 1) H D) of a row), with x the
 * raw projection before the norm, g = dy * gain_p and r = (mean(x^2) + eps)^(-1/2):
 *   dx = r g - r^3 x mean(g x)   (fp32 math, rounded to bf16),
 *   dgain_p = sum over rows and heads of dy x r (fp32, overwritten).
 * x (e.g. mote_qkv_rope_fwd's qk_raw), dy and dx are [rows, parts H D] bf16 with row strides in
 * elements; dx may be dy (in place). D in {32, 64, 96, 128}; rows on 16-byte boundaries.
 * Workspace: mote_head_rms_norm_bwd_workspace() bytes (per-workgroup dgain partials, added in a
 * fixed order: dgain is bitwise reproducible); its contents on entry do not matter.
 * ------------------------------------------------------------------------------------------------ */
typedef struct mote_head_norm_bwd_args {
  int dtype;             /* MOTE_BF16 */
  int rows, parts, H, D;
  float eps;
  const void* x; int64_t x_sr;
  const void* dy; int64_t dy_sr;
  void* dx; int64_t dx_sr;
  const float* gain0;
  const float* gain1;    /* parts == 2 */
  float* dgain0;
  float* dgain1;         /* parts == 2 */
  void* workspace;
  size_t workspace_bytes;
} mote_head_norm_bwd_args;

size_t mote_head_rms_norm_bwd_workspace(const mote_head_norm_bwd_args* args);
int mote_head_rms_norm_bwd(const mote_head_norm_bwd_args* args, void* stream);

/* ------------------------------------------------------------------------------------------------
 * Output gate of FullRelation._out (bf16): z = y * sigmoid(x wg^T) with the product rounded to bf16,
 * the sigmoid rounded to bf16 and z rounded again (the reference's bf16 ops, relation.py:179-181),
 * in one launch of the prologue's product kernel; s receives the sigmoid for the backward.
 * Replaces: `y * torch.sigmoid(self.wg(x))` of mote/model/relation.py:179-181 (one GEMM and two
 * elementwise passes); `wo` follows on the caller's GEMM library.
 * x, y, z, s: [B * T, D] bf16 rows (the batches back to back); w: [D, D] bf16; D a multiple of 128.
 * ------------------------------------------------------------------------------------------------ */
typedef struct mote_gate_product_args {
  int B, T, D;
  const void* x; int64_t x_sr;
  const void* w; int64_t w_sr;
  const void* y; int64_t y_sr;
  void* z;
  void* s;
  int64_t z_sr;             /* row stride of z and s */
} mote_gate_product_args;

int mote_gate_product(const mote_gate_product_args* args, void* stream);

/* ------------------------------------------------------------------------------------------------
 * Weight gradient of a projection (bf16, fp32 accumulation): dW [N, K] = A^T X, A [M, N] (the
 * output gradient) and X [M, K] (the projection's input) token-major, summed over the M rows and
 * rounded once to bf16; bitwise reproducible. N and K multiples of 128, rows on 16-byte boundaries,
 * a_sr, x_sr below 2^24 elements; M == 0 writes zeros. The workspace holds fp32 partials of the
 * splits of M (mote_wgrad_workspace; 0 bytes when one split serves).
 * Replaces: the weight half of autograd through the projections of FullRelation.heads
 * (mote/model/relation.py:204-215: the stacked [w1; w2; wi] product, dW = dqkv^T x), which the
 * GEMM library runs with its reduction over the token rows.
 * ------------------------------------------------------------------------------------------------ */
typedef struct mote_wgrad_args {
  int dtype;               /* MOTE_BF16 */
  int M, N, K;
  const void* a; int64_t a_sr;
  const void* x; int64_t x_sr;
  void* dw; int64_t dw_sr;
  void* workspace;
  size_t workspace_bytes;
} mote_wgrad_args;

size_t mote_wgrad_workspace(const mote_wgrad_args* args);
int mote_wgrad(const mote_wgrad_args* args, void* stream);

/* ------------------------------------------------------------------------------------------------
 * Skinny product for the decode engine's per-token projections (bf16, fp32 accumulation):
 * y [B, N] = x [B, K] W[N, K]^T rounded to bf16, B <= 16 rows (one new chunk per sequence), N a
 * multiple of 16, K a multiple of 128 and at most 1024; x and W rows on 16-byte boundaries, row
 * strides in elements. B == 0 launches nothing.
 * Replaces: the projections around GraphDecoder._relation_step (F.linear of the stacked
 * [w1; w2; wi] and wo, mote/infer/graph.py:151-187, relation.py:176-182) at decode shapes, where
 * the general GEMM library's launch is most of the cost.
 * ------------------------------------------------------------------------------------------------ */
typedef struct mote_skinny_gemm_args {
  int dtype;               /* MOTE_BF16 */
  int B, N, K;
  const void* x; int64_t x_sr;
  const void* w; int64_t w_sr;
  void* y; int64_t y_sr;
  const unsigned char* run;  /* predicate as in mote_relation_decode_args, or NULL */
  /* Optional side job for the decode step that precedes this launch: xm[b] = the mean of
   * g[b * heads .. b * heads + heads - 1] in head order, b < B (graph.py:186), when xm is not NULL.
   * The decode step's g is complete by then (stream order), so the decode launch needs no count of
   * finished heads for xm. Written only when the launch runs (run). */
  const float* g; float* xm; int heads;
} mote_skinny_gemm_args;

int mote_skinny_gemm(const mote_skinny_gemm_args* args, void* stream);

/* ------------------------------------------------------------------------------------------------
 * Arena rows <-> a host page of the prefix store as strided DMA: one hipMemcpy2DAsync per (layer,
 * kind) plane moves its H head rows of `rows` x D elements at their pitches; no staging copy, no
 * kernel. Replaces: the row copies of the prefix store's _store_rows / hydrate
 * (mote/infer/prefix_cache.py:144-165: `page[..., off:off+take].copy_(arena.rows(c, c+take))` and
 * the reverse). to_page = 1: arena rows [arena_row0, +rows) -> page rows [page_row0, +rows);
 * 0: page -> arena. arena: address of element (plane 0, head 0, row 0, 0) of one sequence; a_plane /
 * a_head: elements between planes / heads (the batched arena: batch * H * capacity * D and
 * capacity * D). page likewise (p_plane = H * page_rows * D, p_head = page_rows * D). elem_bytes: 2
 * or 4. Asynchronous on `stream` (host pages pinned).
 * ------------------------------------------------------------------------------------------------ */
typedef struct mote_page_copy_args {
  int to_page, planes, H, D, elem_bytes, rows;
  void* arena; int64_t a_plane, a_head; int arena_row0;
  void* page; int64_t p_plane, p_head; int page_row0;
} mote_page_copy_args;

int mote_arena_page_copy(const mote_page_copy_args* args, void* stream);

/* ------------------------------------------------------------------------------------------------
 * Chunking either side of the main network (mote/model/dc.py:192-352).
 *
 * mote_chunk_route: per row of the boundary mask (bool / uint8 [B, L], row stride mask_sr bytes),
 * cum[b, t] = number of boundaries in [0, t] (int32 [B, L]), perm[b, :] = the boundary positions in
 * order followed by the other positions in order (int32 [B, L]; the reference's
 * argsort(arange(L) + L * !mask), dc.py:212-213 and :320-322) and num[b] = the row's boundary count
 * (dc.py:209). cu_seqlens (int32 [B + 1], may be NULL) receives 0, num[0], num[0] + num[1], ...: the
 * packed layout of the Relation varlen entry point. No host synchronisation: a caller that needs M
 * on the host (the reference's int(num.max()), dc.py:210) reads num.
 * Replaces: the index computation of ChunkLayer.forward and DeChunkLayer.forward (dc.py:209-214, 320-327).
 * ------------------------------------------------------------------------------------------------ */
typedef struct mote_chunk_route_args {
  int B, L;
  const uint8_t* mask; int64_t mask_sr;
  int32_t* cum;
  int32_t* perm;
  int32_t* num;
  int32_t* cu_seqlens;
} mote_chunk_route_args;

int mote_chunk_route(const mote_chunk_route_args* args, void* stream);

/* mote_chunk_gather: out[b, m] = hidden[b, perm[b, m]] for m < M (M <= L; rows past num[b] are the
 * first non-boundary positions, the reference's padded tail, dc.py:196-199, 214-216). With cu_seqlens
 * given, only rows m < num[b] are written, to out row cu_seqlens[b] + m (o_sb unused): the packed
 * varlen layout. hidden [B, L, D] and out have unit element stride, strides in elements; rows are
 * whole 16-byte units (D % 4 == 0 fp32, D % 8 == 0 bf16) on 16-byte boundaries.
 * Replaces: ChunkLayer.forward's gather (dc.py:214-216). */
typedef struct mote_chunk_gather_args {
  int dtype;
  int B, L, M, D;
  const void* hidden; int64_t h_sb, h_sr;
  const int32_t* perm;
  const int32_t* num;
  const int32_t* cu_seqlens;
  void* out; int64_t o_sb, o_sr;
} mote_chunk_gather_args;

int mote_chunk_gather(const mote_chunk_gather_args* args, void* stream);

/* Backward of mote_chunk_gather: dhidden[b, t] = dout row of t when t was gathered, else 0 (every
 * row of dhidden is written). Same layout rules; dout is [B, M, D] or packed [total, D].
 * Replaces: autograd of torch.gather in ChunkLayer.forward. */
typedef struct mote_chunk_gather_bwd_args {
  int dtype;
  int B, L, M, D;
  const void* dout; int64_t g_sb, g_sr;
  const uint8_t* mask; int64_t mask_sr;
  const int32_t* cum;
  const int32_t* num;
  const int32_t* cu_seqlens;
  void* dhidden; int64_t dh_sb, dh_sr;
} mote_chunk_gather_bwd_args;

int mote_chunk_gather_bwd(const mote_chunk_gather_bwd_args* args, void* stream);

/* mote_dechunk_fwd: DeChunkLayer.forward (dc.py:312-335). p_m = clamp(prob[b, perm[b, m], 1], eps,
 * 1 - eps); z_m = p_m hidden[b, m] + (1 - p_m) z_{m-1} in fp32 (z_{-1} = init[b] or 0), for m <
 * num[b]; out[b, t] = z of the last boundary at or before t (perm, num, cum from mote_chunk_route). Bytes before the first boundary read
 * init when it is given (the decode-state form, dc.py:328-332), else z_0 (dc.py:326). hidden is
 * [B, M, D] (M >= num[b]; rows past num[b] are not read), prob [B, L, 2] (strides in elements), out
 * [B, L, D] in hidden's dtype (out_dtype == dtype). w (fp32 [B, M, D], may be NULL) keeps
 * hidden_m - z_{m-1} for the backward. The arithmetic that produces z_m reads chunks <= m only, in an
 * order fixed by m: outputs are causal bit for bit. The caller updates its state from out[:, L - 1]
 * (dc.py:336-337). D even; rows on 2-element boundaries.
 * Workspace: mote_dechunk_workspace() bytes, contents on entry do not matter. */
typedef struct mote_dechunk_args {
  int dtype;        /* hidden */
  int prob_dtype;
  int out_dtype;
  int B, L, M, D;
  float eps;
  const void* hidden; int64_t h_sb, h_sr;
  const void* prob; int64_t p_sb, p_sr;
  const int32_t* perm;
  const int32_t* num;
  const int32_t* cum;
  const float* init;
  void* out; int64_t o_sb, o_sr;
  float* w;
  void* workspace;
  size_t workspace_bytes;
} mote_dechunk_args;

size_t mote_dechunk_workspace(const mote_dechunk_args* args);
int mote_dechunk_fwd(const mote_dechunk_args* args, void* stream);

/* Backward of mote_dechunk_fwd without init (the training form): with ds_m the sum of dout over the
 * bytes of chunk m, g_m = ds_m + (1 - p_{m+1}) g_{m+1}; dhidden[b, m] = p_m g_m (0 for rows no byte
 * reads), dprob[b, t, 1] = sum_d g_m (hidden_m - z_{m-1}) at the position t of chunk m when eps <=
 * prob <= 1 - eps (the clamp's gradient), every other dprob entry 0 (every entry is written). w is
 * the forward's w; dout and dhidden are in hidden's dtype. Sums over channels and bytes run in a
 * fixed order: reproducible.
 * Replaces: autograd of DeChunkLayer.forward / _ema_chunked (dc.py:236-282, 312-335). */
typedef struct mote_dechunk_bwd_args {
  int dtype;        /* hidden */
  int prob_dtype;
  int dout_dtype;
  int dx_dtype;
  int dprob_dtype;
  int B, L, M, D;
  float eps;
  const void* dout; int64_t g_sb, g_sr;
  const void* hidden; int64_t h_sb, h_sr;
  const void* prob; int64_t p_sb, p_sr;
  const int32_t* perm;
  const int32_t* num;
  const uint8_t* mask; int64_t mask_sr;
  const int32_t* cum;
  const float* w;
  void* dhidden; int64_t dh_sb, dh_sr;
  void* dprob; int64_t dp_sb, dp_sr;
  void* workspace;
  size_t workspace_bytes;
} mote_dechunk_bwd_args;

size_t mote_dechunk_bwd_workspace(const mote_dechunk_bwd_args* args);
int mote_dechunk_bwd(const mote_dechunk_bwd_args* args, void* stream);

/* mote_dechunk_step: one decode byte (dc.py:342-352). For row b with mask[b]: p = clamp(prob[b, 1])
 * (rounded to prob's dtype, then to the state's), cur = hidden[r] where r counts the set mask entries
 * before b; else p = 0, cur = 0. last_value[b] = p cur + (1 - p) last_value[b], every operation
 * rounded to the state's dtype as the reference's eager ops are; out[b] (may be NULL) gets the same.
 * Replaces: DeChunkLayer.step. */
typedef struct mote_dechunk_step_args {
  int prob_dtype, hidden_dtype, state_dtype;
  int B, D;
  float eps;
  const uint8_t* mask;
  const void* prob; int64_t p_sr;
  const void* hidden; int64_t h_sr;
  void* last_value; int64_t l_sr;
  void* out; int64_t o_sr;
} mote_dechunk_step_args;

int mote_dechunk_step(const mote_dechunk_step_args* args, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* MOTE_RELATION_H */
