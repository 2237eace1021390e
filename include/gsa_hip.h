/*
 * gsa_hip.h -- C ABI of libgsa_hip.so, the MI355X (gfx950) kernels of the
 * Gated Sparse Attention (GSA) layer forward.
 *
 * Each entry point replaces one step of the reference's optimized forward
 * (gsa_triton/gsa_opt.py); the reference line it replaces is cited above it.
 *
 * Conventions
 *  - Plain pointers and sizes; no framework types.  Device pointers are HIP
 *    device pointers; `stream` is a hipStream_t (NULL = the null stream).
 *  - Tensors are [B, T, ...] with the innermost dimensions (heads, then
 *    elements) contiguous; each tensor is described by its pointer and its
 *    batch and row strides, in elements.  Strided views into one fused
 *    projection output are therefore accepted without copies.  The indexer
 *    entry points address 16 rows of k_idx with 32-bit offsets: they reject
 *    (GSA_ERR_SHAPE) a negative k_idx row stride or one whose 16 rows span
 *    2 GiB or more.
 *  - dtype is GSA_DTYPE_BF16 or GSA_DTYPE_F32 for every floating tensor of a
 *    call (indices and counts are int32, masks uint8, scores and bias fp32).
 *  - Ownership: the caller owns every buffer.  The library never allocates,
 *    frees or retains device memory and never synchronises; every call is
 *    enqueued on `stream` and returns.  (The one exception is the static
 *    device array behind gsa_indexer_select_noalloc: it is part of the loaded
 *    code object, one copy per device, and lives until the process ends.)
 *  - Errors: 0 on success; > 0 for argument errors, detected on the host
 *    before anything is enqueued; < 0 is the negated hipError_t of a failed
 *    launch.  gsa_status_string() names every code.
 *  - Thread safety: all entry points are reentrant.
 */
#ifndef GSA_HIP_H
#define GSA_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define GSA_ABI_VERSION 3

#define GSA_DTYPE_F32  0
#define GSA_DTYPE_BF16 1

#define GSA_OK            0
#define GSA_ERR_NULL      1  /* a required pointer is NULL                        */
#define GSA_ERR_SHAPE     2  /* unsupported or inconsistent sizes                 */
#define GSA_ERR_DTYPE     3  /* unknown dtype code                                */
#define GSA_ERR_ALIGN     4  /* pointer or stride breaks the vector-load alignment */
#define GSA_ERR_K         5  /* k out of range (k < 1, k > keys, or too large)     */
#define GSA_ERR_FLAGS     6  /* unknown flag or order code                         */
#define GSA_ERR_SCRATCH   7  /* sizes exceed gsa_indexer_select_noalloc's static scratch */

/* Order of gsa_topk_select's output */
#define GSA_ORDER_INDEX_ASC  0  /* valid indices ascending, then invalid ones ascending */
#define GSA_ORDER_SCORE_DESC 1  /* by (score desc, index asc): torch.topk's sorted order */

/* Flags of gsa_sparse_attn */
#define GSA_ATTN_ROPE_Q   1  /* q is pre-RoPE: apply RoPE with cos/sin in the prologue  */
#define GSA_ATTN_OUT_GATE 2  /* multiply the output by sigmoid(og) (the G1 output gate) */
#define GSA_ATTN_MASKS_READY 4  /* gsa_dense_attn: ws already holds gsa_dense_lane_masks of bits */
#define GSA_ATTN_ROPE_HALVES 8  /* gsa_dense_attn with GSA_ATTN_ROPE_Q: cos is the packed table below */

/* Largest k_eff of gsa_topk_select in GSA_ORDER_SCORE_DESC order. */
#define GSA_TOPK_DESC_MAX_K 4096

int gsa_abi_version(void);
const char* gsa_status_string(int status);

/*
 * Fused gated lightning indexer, full score matrix.
 * Replaces fused_gated_indexer (gsa_triton/gsa_opt.py:143-176) and its kernel
 * (gsa_opt.py:38-140); semantics of GatedLightningIndexer.forward
 * (gsa_triton/gsa_ref.py:97-126):
 *   scores[b,i,j] = sum_h sigmoid(w[b,i,h]) * sigmoid(scale*<q[b,i,h,:], k[b,j,:]> + bias[h])
 *   for j <= i (or every j when causal == 0), -inf otherwise.
 * q_idx [B,T,Hi,di], k_idx [B,T,di], w [B,T,Hi] in dtype; bias fp32 [Hi];
 * scores fp32 [B,T,T] with strides (s_sb, s_st), unit column stride.
 * Supported: Hi == 4, di == 64.
 */
int gsa_indexer_scores(const void* q_idx, int64_t q_sb, int64_t q_st,
                       const void* k_idx, int64_t k_sb, int64_t k_st,
                       const void* w, int64_t w_sb, int64_t w_st,
                       const float* bias, float scale,
                       int B, int T, int Hi, int di, int causal, int dtype,
                       float* scores, int64_t s_sb, int64_t s_st,
                       void* stream);

/*
 * Exact per-row top-k of an fp32 score matrix.
 * Replaces AdaptiveTopKSelector.forward (gsa_triton/gsa_opt.py:473-483,
 * gsa_triton/gsa_ref.py:138-150) and the ascending re-sort of the optimized
 * forward (gsa_opt.py:674-677).
 * Row r of scores [B,T,Tkv] selects the k_eff largest after mapping -inf to
 * -1e9 (NaN ranks above +inf); ties at the k-th value go to the lowest
 * indices.  An entry is valid when its score is not -inf.
 *   order GSA_ORDER_INDEX_ASC : idx_out row = valid selected ascending, then
 *                               invalid selected ascending; count = #valid.
 *   order GSA_ORDER_SCORE_DESC: idx_out row sorted by (score desc, index asc);
 *                               k_eff <= GSA_TOPK_DESC_MAX_K.
 * idx_out int32 [B,T,k_eff] contiguous; count_out int32 [B,T] (nullable);
 * mask_out uint8 [B,T,k_eff] (nullable): 1 where the entry is valid.
 */
int gsa_topk_select(const float* scores, int64_t s_sb, int64_t s_st,
                    int B, int T, int Tkv, int k_eff, int order,
                    int32_t* idx_out, int32_t* count_out, uint8_t* mask_out,
                    void* stream);

/*
 * gsa_topk_select with the variance-based per-row k of gsa_explained.ipynb:
 * 577-592 (the rule AdaptiveTopKSelector, gsa_triton/gsa_opt.py:466-483,
 * keeps k_min for but does not apply).  var_out[r] = population variance of
 * row r's finite scores (two passes: mean, then squared deviations); with avg
 * their mean over all B*T rows,
 *   k_out[r] = min(clamp(floor(k_base * max(avg,1e-6) / max(var_out[r],1e-6)), k_min, k_max), Tkv).
 * Row r then selects k_out[r] entries as gsa_topk_select does; output rows
 * are W = min(k_max, Tkv) wide and entries k_out[r] .. W-1 are index 0 with
 * mask 0.  idx_out int32 [B,T,W]; count_out (nullable), k_out int32 [B*T];
 * var_out float [B*T]; mask_out uint8 [B,T,W] (nullable).  Three launches in
 * stream order.  GSA_ORDER_SCORE_DESC needs W <= GSA_TOPK_DESC_MAX_K.
 */
int gsa_topk_select_adaptive(const float* scores, int64_t s_sb, int64_t s_st,
                             int B, int T, int Tkv, int k_base, int k_min, int k_max, int order,
                             int32_t* idx_out, int32_t* count_out, uint8_t* mask_out,
                             int32_t* k_out, float* var_out,
                             void* stream);

/*
 * Indexer and selector fused.
 * Replaces the indexer track of the optimized forward (gsa_triton/gsa_opt.py:
 * 663-677: fused_gated_indexer + AdaptiveTopKSelector + ascending sort).
 * Selects exactly what gsa_indexer_scores followed by gsa_topk_select
 * (causal) select.  Always writes the selection as a bitmask: bits uint32
 * [B,T,W] (strides b_sb, b_st; W = 2*ceil(T/64) words per row; bit j of row
 * t set iff key j is selected; 8-byte aligned rows), the form gsa_dense_attn
 * takes.  When idx_out and count_out are given it also writes, like
 * GSA_ORDER_INDEX_ASC: idx_out int32 [B,T,k_eff] = row t's min(t+1, k_eff)
 * selected keys ascending, followed by t+1, t+2, ...; count_out int32 [B,T].
 * No score is stored: a sample of every fourth key tile places a band around
 * each row's k-th score, one exact pass writes the sure winners into the mask
 * and keeps the band's keys as candidates, and a row whose counts do not
 * prove the band is selected by an exact radix select over recomputed scores.
 * The candidates stay in LDS.  ws: caller-provided device workspace of at
 * least gsa_indexer_select_workspace_bytes(B, T) bytes (16-byte aligned),
 * overwritten by each call: 512 bytes of store slots per 16-row group
 * (B * ceil(T/16) * 512 bytes).
 * Supported: Hi == 4, di == 64, 1 <= k_eff <= T <= 65536.
 */
size_t gsa_indexer_select_workspace_bytes(int B, int T);

int gsa_indexer_select(const void* q_idx, int64_t q_sb, int64_t q_st,
                       const void* k_idx, int64_t k_sb, int64_t k_st,
                       const void* w, int64_t w_sb, int64_t w_st,
                       const float* bias, float scale,
                       int B, int T, int Hi, int di, int k_eff, int dtype,
                       uint32_t* bits, int64_t b_sb, int64_t b_st,
                       int32_t* idx_out, int32_t* count_out,
                       void* ws, size_t ws_bytes,
                       void* stream);

/*
 * gsa_indexer_select without a workspace argument, for callers that cannot
 * allocate (code under HIP graph capture, serving loops, harnesses that forbid
 * hipMalloc).  No counterpart in the reference.  Same arguments, outputs and
 * checks as gsa_indexer_select minus ws/ws_bytes; its launches use a static
 * device array of gsa_indexer_select_noalloc_max_bytes() bytes (4 MiB; one
 * copy per device, held until the process ends) instead, so it accepts only
 * gsa_indexer_select_workspace_bytes(B, T) <= that, i.e. B * ceil(T/16) <=
 * 8192 (GSA_ERR_SCRATCH otherwise, before anything is enqueued).  It calls no
 * allocator.  The first call on a device looks the array's address up on
 * that device.  Every call on one device shares that device's array: calls
 * that overlap on one device race on it (the selector only stores discarded
 * values there, but no result is promised for overlapping calls).
 */
size_t gsa_indexer_select_noalloc_max_bytes(void);

int gsa_indexer_select_noalloc(const void* q_idx, int64_t q_sb, int64_t q_st,
                               const void* k_idx, int64_t k_sb, int64_t k_st,
                               const void* w, int64_t w_sb, int64_t w_st,
                               const float* bias, float scale,
                               int B, int T, int Hi, int di, int k_eff, int dtype,
                               uint32_t* bits, int64_t b_sb, int64_t b_st,
                               int32_t* idx_out, int32_t* count_out,
                               void* stream);

/*
 * The fused indexer + exact top-k with a per-row k from the score variance:
 * the variance-based adaptive rule of gsa_explained.ipynb:577-592, which the
 * reference's AdaptiveTopKSelector (gsa_triton/gsa_opt.py:466-483) stores
 * k_min for but does not apply.  With var_t the population variance of row
 * t's causal scores (keys j <= t) and avg the mean of var_t over all B*T rows,
 *   k_t = min(clamp(floor(k_base * max(avg,1e-6) / max(var_t,1e-6)), k_min, k_max), T)
 * and row t selects its k_t largest causal scores exactly as gsa_indexer_select
 * does for a fixed k (ties at the k-th value to the lowest indices).
 * Outputs: bits as gsa_indexer_select; optionally idx_out int32
 * [B,T,min(k_max,T)] and count_out int32 [B,T] (count = min(t+1, k_t);
 * row t: the count selected keys ascending, then t+1, t+2, ... up to entry
 * k_t - 1 (present only when t+1 < k_t), then index 0 up to the width, so
 * every entry lies in [0, T)); optionally k_out int32 [B*T] (k_t) and var_out float [B*T] (var_t).
 * Three launches on the stream (sample histograms + variances; the global
 * mean and k_t; the select), all in stream order.  ws: at least
 * gsa_indexer_select_adaptive_workspace_bytes(B, T) bytes (16-byte aligned):
 * gsa_indexer_select's workspace, the per-row sample histograms kept between
 * the launches (B * ceil(T/16) * 32 KiB), and room for var and k.
 * Supported: Hi == 4, di == 64, 1 <= k_min <= k_max, k_base >= 1,
 * T <= 65536.
 */
size_t gsa_indexer_select_adaptive_workspace_bytes(int B, int T);

/*
 * Test hook, no counterpart in the reference: while on != 0, every row of
 * gsa_indexer_select / gsa_indexer_select_adaptive that has more causal keys
 * than its k takes the exact fallback path (radix select over recomputed
 * scores) instead of the sampled band, so that tests can check that path on
 * ordinary inputs.  Process-wide; returns the previous setting.
 */
int gsa_debug_force_select_fallback(int on);

int gsa_indexer_select_adaptive(const void* q_idx, int64_t q_sb, int64_t q_st,
                                const void* k_idx, int64_t k_sb, int64_t k_st,
                                const void* w, int64_t w_sb, int64_t w_st,
                                const float* bias, float scale,
                                int B, int T, int Hi, int di,
                                int k_base, int k_min, int k_max, int dtype,
                                uint32_t* bits, int64_t b_sb, int64_t b_st,
                                int32_t* idx_out, int32_t* count_out,
                                int32_t* k_out, float* var_out,
                                void* ws, size_t ws_bytes,
                                void* stream);

/*
 * Producer pass over the projection output: RoPE on k and the G2 value gate.
 * Replaces gsa_triton/gsa_opt.py:685-697 (v * sigmoid(vg), RoPE on k).
 *   k_out = k*cos + rotate_half(k)*sin,  v_out = v * sigmoid(vg)
 * with each op rounded in dtype as the reference rounds it.  Either half may
 * be skipped: k == NULL skips RoPE (cos, sin, k_out unused), v == NULL skips
 * the gate (vg, v_out unused); the same halves back apply_rotary_pos_emb
 * (gsa_opt.py:396-401) and ValueGate/OutputGate (gsa_opt.py:486-507).
 * k, v, vg [B,T,H,d]; cos, sin [T,d] (row stride cs_st) in dtype;
 * k_out, v_out contiguous [B,T,H,d].  Supported: d == 128, 1 <= H <= 64.
 */
int gsa_prologue(const void* k, int64_t k_sb, int64_t k_st,
                 const void* v, int64_t v_sb, int64_t v_st,
                 const void* vg, int64_t g_sb, int64_t g_st,
                 const void* cos, const void* sin, int64_t cs_st,
                 int B, int T, int H, int d, int dtype,
                 void* k_out, void* v_out,
                 void* stream);

/*
 * Sparse attention over per-row selected keys (gather, online softmax).
 * Replaces fused_sparse_attention (gsa_triton/gsa_opt.py:349-383) and its
 * kernel (gsa_opt.py:187-346); with GSA_ATTN_ROPE_Q it also applies RoPE to q
 * (gsa_opt.py:692-697) and with GSA_ATTN_OUT_GATE the G1 gate
 * (gsa_opt.py:699-701, 719-721).  Semantics of sparse_attention_ref
 * (gsa_triton/gsa_ref.py:202-238): for every (b,t,h),
 *   out = sum_m softmax_m(scale * <q, k[idx_m]>) v[idx_m]
 * over the valid entries m (all masked -> 0).  Entry m of row (b,t) is valid
 * when m < count[b,t] (count may be NULL: all k_sel entries) and
 * mask[b,t,m] != 0 (mask may be NULL).  Indices are clamped to [0, Tkv-1].
 * q [B,T,H,d], k, v [B,Tkv,H,d], og [B,T,H,d], out [B,T,H,d] in dtype;
 * idx int32 and mask uint8 share the strides (i_sb, i_st); count int32 [B,T].
 * Supported: d == 128, 1 <= H <= 64.
 */
int gsa_sparse_attn(const void* q, int64_t q_sb, int64_t q_st,
                    const void* k, int64_t k_sb, int64_t k_st,
                    const void* v, int64_t v_sb, int64_t v_st,
                    const int32_t* idx, int64_t i_sb, int64_t i_st, int k_sel,
                    const int32_t* count, const uint8_t* mask,
                    const void* og, int64_t o_sb, int64_t o_st,
                    const void* cos, const void* sin, int64_t cs_st,
                    void* out, int64_t out_sb, int64_t out_st,
                    int B, int T, int Tkv, int H, int d, float scale,
                    int dtype, int flags,
                    void* stream);

/*
 * Producer for the block-dense attention: RoPE on k (k == NULL skips it) and
 * the G2 gate with V written transposed.  Replaces gsa_triton/gsa_opt.py:
 * 685-697 like gsa_prologue, with the value output laid out for
 * gsa_dense_attn: vt[b][h][d][j] = (v * sigmoid(vg))[b][j][h][d] for
 * j < T, 0 for T <= j < ldv (ldv a multiple of 64, >= T).  bf16 only.
 * k_out contiguous [B,T,H,d]; vt contiguous [B,H,d,ldv].
 */
int gsa_prologue_vt(const void* k, int64_t k_sb, int64_t k_st,
                    const void* v, int64_t v_sb, int64_t v_st,
                    const void* vg, int64_t g_sb, int64_t g_st,
                    const void* cos, const void* sin, int64_t cs_st,
                    int B, int T, int H, int d, int dtype,
                    void* k_out, void* vt, int ldv,
                    void* stream);

/*
 * Selection bitmask: bits[b][t][j/32] bit j%32 is set when key j is a valid
 * selected entry of row (b,t) -- entry m valid as in gsa_sparse_attn (m <
 * count, mask != 0), index clamped to [0, Tkv-1] like the reference
 * (gsa_triton/gsa_ref.py:196); a key selected twice is set once.
 * bits uint32 [B,T,W] with W = 2*ceil(Tkv/64) (8-byte aligned rows).
 * Replaces nothing in the reference: it is the mask form of the selection
 * (gsa_opt.py:671-677) that gsa_dense_attn consumes.
 */
int gsa_selection_mask(const int32_t* idx, int64_t i_sb, int64_t i_st, int k_sel,
                       const int32_t* count, const uint8_t* mask,
                       int B, int T, int Tkv, uint32_t* bits, int64_t b_sb, int64_t b_st,
                       void* stream);

/*
 * Block-dense sparse attention on MFMA: the function of gsa_sparse_attn
 * (fused_sparse_attention, gsa_triton/gsa_opt.py:349-383, with the optional
 * RoPE(q) and G1 gate of gsa_opt.py:692-701,719-721) computed over whole
 * 64-key tiles with the selection applied as a bitmask (bits as written by
 * gsa_indexer_select or gsa_selection_mask).
 * q, out, og [B,T,H,d]; k [B,Tkv,H,d] (RoPE'd); vt [B,H,d,ldv] as written by
 * gsa_prologue_vt (strides vt_sb, vt_sh per batch and head; rows of ldv).
 * causal != 0: key tiles after a query block's last row are skipped (the
 * selection must then be causal; a block holds 256 query rows).
 * ws: caller-provided device workspace of at least
 * gsa_dense_attn_workspace_bytes(B, T, Tkv) bytes (16-byte aligned; 1 KiB
 * of mask operands per 32 query rows and 64 keys), overwritten by each call
 * -- or, with GSA_ATTN_MASKS_READY, the mask operands gsa_dense_lane_masks
 * wrote there for the same bits, B, T, Tkv and causal (then bits is not
 * read).  bf16 only; d == 128, 1 <= H <= 64; row strides k_st, q_st, out_st and
 * (with their flags) o_st and cs_st at most 2^24 elements, else GSA_ERR_SHAPE.
 * GSA_ATTN_ROPE_HALVES (with GSA_ATTN_ROPE_Q): cos points to a packed table
 * whose row t holds cos[t][0:64] then sin[t][0:64] (128 elements, row stride
 * cs_st) and sin is not read.  It serves tables whose entries d and d+64 are
 * equal, as RotaryEmbedding builds them (cat(freqs, freqs),
 * gsa_triton/gsa_ref.py:52-56; gsa_opt.py:404-429); the output is then
 * bit-identical to the call with the full cos and sin tables.
 */
size_t gsa_dense_attn_workspace_bytes(int B, int T, int Tkv);

/*
 * The first step of gsa_dense_attn on its own: the selection bitmask ->
 * the attention kernel's mask operands (4 bits per query row and key: the
 * e2m1 operand of the MFMA that starts each score tile), into ws (same size
 * and alignment as gsa_dense_attn's workspace).  Lets a caller build them
 * on another stream, beside other work, and pass GSA_ATTN_MASKS_READY.
 * causal != 0: only the key tiles a causal gsa_dense_attn reads (up to the
 * last row of each query block) are built; such masks serve causal calls
 * only.  causal == 0: every tile (serves both).
 * No counterpart in the reference: part of this library's dense attention.
 */
int gsa_dense_lane_masks(const uint32_t* bits, int64_t b_sb, int64_t b_st,
                         int B, int T, int Tkv, int causal, void* ws, size_t ws_bytes, void* stream);

/*
 * gsa_prologue_vt (RoPE(k) and v*sigmoid(vg) as V^T: gsa_opt.py:685-697) and
 * gsa_dense_lane_masks in one launch, their blocks interleaved so that both
 * run side by side; same arguments, checks and outputs as the two calls.
 * For callers that build the lane masks on the producer's stream right
 * before gsa_dense_attn (no second stream, no join).
 */
int gsa_prologue_vt_lane_masks(const void* k, int64_t k_sb, int64_t k_st,
                               const void* v, int64_t v_sb, int64_t v_st,
                               const void* vg, int64_t g_sb, int64_t g_st,
                               const void* cos, const void* sin, int64_t cs_st,
                               int B, int T, int H, int d, int dtype,
                               void* k_out, void* vt, int ldv,
                               const uint32_t* bits, int64_t b_sb, int64_t b_st, int Tkv,
                               int causal, void* ws, size_t ws_bytes, void* stream);

int gsa_dense_attn(const void* q, int64_t q_sb, int64_t q_st,
                   const void* k, int64_t k_sb, int64_t k_st,
                   const void* vt, int64_t vt_sb, int64_t vt_sh, int ldv,
                   const uint32_t* bits, int64_t b_sb, int64_t b_st,
                   const void* og, int64_t o_sb, int64_t o_st,
                   const void* cos, const void* sin, int64_t cs_st,
                   void* out, int64_t out_sb, int64_t out_st,
                   int B, int T, int Tkv, int H, int d, float scale,
                   int dtype, int flags, int causal,
                   void* ws, size_t ws_bytes,
                   void* stream);

/*
 * Main projection GEMM with the producer fused into its epilogue.
 * Replaces the phase-1 projection GEMM and its split (gsa_triton/gsa_opt.py:
 * 629-638) together with the track-B producer steps that follow it: the
 * value gate v*sigmoid(vg) (gsa_opt.py:685-690) and RoPE(k) (gsa_opt.py:
 * 692-697) -- the producer fusion listed as future work in
 * gsa_triton/README.md:424-433.  RoPE(q) and the output gate stay in
 * gsa_dense_attn, which consumes every output here.
 *
 * gsa_proj_pack (once per weight update): w [5D, D] bf16 (row stride w_st)
 * holds the q, k, v, value-gate and output-gate projection rows in that
 * order, bias [5D] bf16 or NULL (zeros); writes the permuted, tiled weight
 * w_packed (gsa_proj_packed_bytes(D, H) bytes, 16-byte aligned) and the
 * fp32 bias bias_packed [5D].  Supported: D == 128*H, D % 256 == 0 (even H).
 *
 * gsa_proj_fused: x [B*T, D] bf16 rows (stride x_st, multiple of 8) ->
 *   q  [B*T, D] rows (stride q_st):  bf16(x W_q^T + b_q)
 *   og [B*T, D] rows (stride og_st): bf16(x W_og^T + b_og)
 *   k_out [B,T,H,128] contiguous:    RoPE(bf16(x W_k^T + b_k)) with cos/sin
 *                                    [>=T, 128] bf16 (row stride cs_st)
 *   vt [B,H,128,ldv] contiguous:     (bf16(x W_v^T + b_v) *
 *                                    bf16(sigmoid(bf16(x W_vg^T + b_vg))))^T,
 *                                    keys [T, ldv) zero
 * with the rounding points of the unfused path (projection rounded to bf16,
 * then gsa_prologue_vt's steps).  Needs T % 64 == 0, ldv >= T, ldv % 64 == 0.
 */
size_t gsa_proj_packed_bytes(int D, int H);
int gsa_proj_pack(const void* w, int64_t w_st, const void* bias, int D, int H, int dtype,
                  void* w_packed, float* bias_packed, void* stream);
int gsa_proj_fused(const void* x, int64_t x_st, int B, int T, int D, int H, int dtype,
                   const void* w_packed, const float* bias_packed,
                   const void* cos, const void* sin, int64_t cs_st,
                   void* q, int64_t q_st, void* og, int64_t og_st,
                   void* k_out, void* vt, int ldv, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* GSA_HIP_H */
