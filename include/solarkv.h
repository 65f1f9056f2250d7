/*
 * solarkv.h — C ABI of libsolarkv.so, the MI355X (gfx950) block-causal KV-cache path.
 *
 * Every entry point is stream-ordered (it enqueues work on `stream` and returns without a
 * host synchronisation) and returns 0 on success or a negative SKV_E_* code; skv_last_error()
 * then names the failing argument.  The library never allocates device memory: all tensors,
 * including the scratch two faster paths use, are owned by the caller, and pointers are device
 * addresses unless the parameter says "host".  The scratch ("workspace") paths are taken only
 * through the descriptor entry points when the caller passes a workspace at least as large as
 * the query functions report:
 *   - attention over an under-filled grid takes the balanced key split (skv_attention_plan:
 *     2 x n_cu x 256 rows x 130 floats, 68 MB on 256 CUs);
 *   - an fp8 append of a chunk with fewer than 4 (frame, batch, head, K|V) units per CU takes
 *     the one-pass slice kernel (bf16 sources, no K norm, 8-byte aligned workspace: a 128 B
 *     header + 512 B per unit) or else the tile-grid kernels (one float per 64-token tile);
 *     skv_append_workspace_size reports the larger of the two.
 * Without a workspace the same calls run the unsplit kernels (same results up to fp32
 * summation order for attention; bit-identical for the append).  A workspace is read and
 * written by the launch on `stream` only, so one workspace serves any number of calls on one
 * stream; calls on different streams need different workspaces.
 *
 * Frame-slot pool layout (one pair of pools per transformer layer):
 *   K pool  [n_slots][B][H][Tp][D]   row-major keys of each frame, D contiguous
 *   V pool  [n_slots][B][H][D][Tp]   values stored transposed (tokens contiguous per channel)
 *   scales  [n_slots][B][H] float    fp8 pools only: dequantisation scale = absmax / 448
 * T is the frame's token count and Tp = T rounded up to a multiple of 64; rows T..Tp-1 of a
 * slot are zero so that a 64-key tile never straddles two frames.
 *
 * Token-major tensors (new K/V, queries, outputs, gathered views) are [B][L][H][D] with
 * element strides (sb, st, sh) and a unit stride on D — the reference layout
 * (solar/backends/wan22/runtime/stage2.py:1776-1793, attention.py:56-60).
 */
#ifndef SOLARKV_H
#define SOLARKV_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef void* skv_stream_t; /* a hipStream_t; NULL = the null stream */

enum skv_dtype {
  SKV_F32 = 0,
  SKV_BF16 = 1,
  SKV_FP8_E4M3 = 2, /* OCP e4m3fn, pools only */
  SKV_F16 = 3       /* IEEE binary16: f16 pools filled from f16 sources (plain append, no
                       norm / RoPE / PRoPE), gathered, and attended with f16 MFMAs (plain
                       attention; queries and outputs f16 or f32) */
};

enum skv_mask_mode {
  SKV_MASK_NONE = 0,        /* every query sees every key of the frame list */
  SKV_MASK_CHUNK_CAUSAL = 1 /* query at position p sees keys < min((p / chunk + 1) * chunk, n_keys) */
};

enum skv_status {
  SKV_OK = 0,
  SKV_E_ARG = -1,         /* bad pointer, size, stride or dtype */
  SKV_E_UNSUPPORTED = -2, /* valid request this build does not implement (e.g. head_dim != 128) */
  SKV_E_LAUNCH = -3       /* the HIP launch itself failed */
};

#define SKV_MAX_APPEND_FRAMES 64
#define SKV_MAX_FRAMES 256
#define SKV_MAX_SEGMENTS 64

/* Library version as an integer (major * 10000 + minor * 100 + patch). */
int skv_version(void);

/* Message of the last failing call on this host thread ("" if none). */
const char* skv_last_error(void);

/*
 * skv_append — write n_frames whole frames of new K/V into pool slots.
 * Replaces the slice assignments of the reference cache update:
 *   causal_model.py:1074-1080 (rolling), :1115-1121 (direct), :2894-2898 / :2910-2914 (commit).
 * Frame f (0 <= f < n_frames) is source tokens [(src_frame0 + f) * T, (src_frame0 + f + 1) * T)
 * of k_new / v_new and goes to slot dst_slots[f] (host array, copied into the launch).
 * pool_dtype SKV_FP8_E4M3 quantises with one scale per (slot, b, h):
 *   scale = absmax / 448, code = e4m3fn(clamp(x * (448 / absmax), -448, 448)), 0 if absmax == 0;
 * k_scale / v_scale must then be non-NULL, otherwise they are ignored.
 */
int skv_append(const void* k_new, const void* v_new, int src_dtype, int64_t src_sb,
               int64_t src_st, int64_t src_sh, int src_frame0, void* k_pool, void* v_pool,
               float* k_scale, float* v_scale, int pool_dtype, int n_slots,
               const int32_t* dst_slots /* host */, int n_frames, int batch, int heads,
               int head_dim, int frame_tokens, skv_stream_t stream);

/*
 * skv_gather — materialise pool frames slots[0..n_frames) as contiguous token-major K and V
 * [B][n_frames * T][H][D] (the reference's torch.cat of cached frames:
 * causal_model.py:1155-1156, memory_retrieval.py:79-86).  out_dtype must equal pool_dtype
 * (an fp8 pool is copied as raw codes; its scales stay in the scale arrays).
 */
int skv_gather(const void* k_pool, const void* v_pool, int pool_dtype, int n_slots,
               const int32_t* slots /* host */, int n_frames, int batch, int heads, int head_dim,
               int frame_tokens, void* k_out, void* v_out, int64_t out_sb, int64_t out_st,
               int64_t out_sh, skv_stream_t stream);

/*
 * skv_attention — out = softmax(q kᵀ · softmax_scale) v over the keys of the frame list
 * frame_slots[0..n_frames) (host array) taken in order, i.e. n_keys = n_frames * T.
 * Replaces attention(q, cat[sink, local]) of causal_model.py:1135-1226 → attention.py:141-188
 * (mask_mode NONE) and the chunk-causal FlexAttention of causal_model.py:474-534, :984-989
 * (mask_mode CHUNK_CAUSAL, query i at position q_pos0 + i).
 * q and out are token-major [B][Lq][H][D]; q_dtype in {F32, BF16} (F32 is rounded to bf16 as the
 * reference's flash path does, attention.py:69-73), out_dtype == q_dtype.  Pools may be F32,
 * BF16 or FP8_E4M3 (k_scale / v_scale required for FP8).  Compute: bf16 (fp8 for FP8 pools)
 * matrix-core products with fp32 accumulation and an fp32 online softmax.
 */
int skv_attention(const void* q, int q_dtype, int64_t q_sb, int64_t q_st, int64_t q_sh,
                  const void* k_pool, const void* v_pool, const float* k_scale,
                  const float* v_scale, int pool_dtype, int n_slots,
                  const int32_t* frame_slots /* host */, int n_frames, int batch, int heads,
                  int head_dim, int q_len, int frame_tokens, float softmax_scale, int mask_mode,
                  int64_t q_pos0, int64_t chunk_tokens, void* out, int64_t out_sb,
                  int64_t out_st, int64_t out_sh, skv_stream_t stream);

/*
 * RoPE on load (pre-RoPE caches, as the reference keeps them).  The reference re-ropes the
 * visible window in float64 on every forward: sink frames at temporal positions 0.., local
 * frames and the query chunk at window-relative positions (causal_model.py:791-876 via
 * echorope_apply :88-197; table model.py:28-35, split causal_model.py:1855-1866: per head 22
 * temporal, 21 height and 21 width complex pairs (2i, 2i+1)).  Here:
 *
 * skv_append_rope — skv_append for bf16/f32 pools that also writes K with its height/width pairs
 * rotated (token t of a frame sits at h = t / grid_w, w = t % grid_w) into kr_pool (same layout
 * as k_pool).  rope_hw (device, float32) holds cos, sin per (h, pair) for h < grid_h, then per
 * (w, pair) for w < grid_w: [(grid_h + grid_w) * 21 * 2].  grid_h * grid_w == frame_tokens.
 * k_pool / v_pool receive the raw frames exactly as skv_append writes them.
 */
int skv_append_rope(const void* k_new, const void* v_new, int src_dtype, int64_t src_sb,
                    int64_t src_st, int64_t src_sh, int src_frame0, void* k_pool, void* v_pool,
                    int pool_dtype, int n_slots, const int32_t* dst_slots /* host */,
                    int n_frames, int batch, int heads, int head_dim, int frame_tokens,
                    void* kr_pool, const float* rope_hw, int grid_h, int grid_w,
                    skv_stream_t stream);

/*
 * skv_attention_rope — skv_attention (bf16 pools) over keys from kr_pool (written by
 * skv_append_rope) with un-roped queries: the kernel rotates each query's height/width pairs
 * (rope_hw) and, for every key frame j, its temporal pairs by the angle of (query frame f, key
 * frame j): rope_t (device, float32) = cos, sin of (p_query[f] - p_key[j]) * theta^(-2i/44) per
 * [f][j][i], i < 22, f < n_qframes (q_len == n_qframes * frame_tokens, query row r is frame
 * r / T, token r % T).  Scores equal those of queries and keys roped at p_query / p_key.
 */
int skv_attention_rope(const void* q, int q_dtype, int64_t q_sb, int64_t q_st, int64_t q_sh,
                       const void* kr_pool, const void* v_pool, int pool_dtype, int n_slots,
                       const int32_t* frame_slots /* host */, int n_frames, int batch,
                       int heads, int head_dim, int q_len, int frame_tokens,
                       float softmax_scale, int mask_mode, int64_t q_pos0,
                       int64_t chunk_tokens, void* out, int64_t out_sb, int64_t out_st,
                       int64_t out_sh, const float* rope_hw, int grid_h, int grid_w,
                       const float* rope_t, int n_qframes, skv_stream_t stream);

/*
 * Fused PRoPE on top of RoPE on load (camera-conditioned caches).  The reference's fused mode
 * keeps raw K/V plus a camera cache with the same token layout, re-ropes the window and then
 * applies PRoPE: q' = P_qᵀ q, k' = P_k⁻¹ k, v' = P_k⁻¹ v on every group of 4 head channels
 * (P = lift(K_norm) · viewmat of the token's camera), attends, and maps the output back with P_q
 * (causal_model.py:585-651, :1170-1199 → camera_prope.py:93-261; camera cache
 * causal_model.py:1948-2075).  Cameras are per latent frame (the data path expands one camera
 * per frame to every token, data.py:516-530).  Matrices are row-major 4x4 float32.
 *
 * skv_append_prope — skv_append_rope (bf16 pools) that also applies P_k⁻¹ of each written frame's
 * camera, kv_xform[f][b] (device, [n_frames][batch][16]): kx_pool receives K with its
 * height/width pairs rotated and then P_k⁻¹ on channel groups 11..31 (channels 44..127; groups
 * 0..10 hold temporal pairs and stay raw), vx_pool receives P_k⁻¹ v on every group (V layout).
 * k_pool / v_pool receive the raw frames exactly as skv_append writes them.
 */
int skv_append_prope(const void* k_new, const void* v_new, int src_dtype, int64_t src_sb,
                     int64_t src_st, int64_t src_sh, int src_frame0, void* k_pool, void* v_pool,
                     int pool_dtype, int n_slots, const int32_t* dst_slots /* host */,
                     int n_frames, int batch, int heads, int head_dim, int frame_tokens,
                     void* kx_pool, void* vx_pool, const float* rope_hw, int grid_h, int grid_w,
                     const float* kv_xform, skv_stream_t stream);

/*
 * skv_attention_prope — skv_attention_rope over kx_pool / vx_pool (written by skv_append_prope)
 * with un-roped queries; frame_tokens >= 64.  Device tables, for query frame f of stream b and
 * key frame j of the list:
 *   q_xform_t [b][j][f][11][16]  W = R_k(p_k)ᵀ (P_q P_k⁻¹)ᵀ R_q(p_q) per temporal group g < 11,
 *                                R = the group's two temporal RoPE rotations (angles p·θ^(-2i/44))
 *   q_xform_s [b][f][16]         P_qᵀ, applied to the spatial groups after their RoPE rotation
 *   out_xform [b][f][16]         P_q, applied to every group of the output
 * Scores equal those of the reference's RoPE-then-PRoPE queries and keys; the output is P_q o.
 */
int skv_attention_prope(const void* q, int q_dtype, int64_t q_sb, int64_t q_st, int64_t q_sh,
                        const void* kx_pool, const void* vx_pool, int pool_dtype, int n_slots,
                        const int32_t* frame_slots /* host */, int n_frames, int batch,
                        int heads, int head_dim, int q_len, int frame_tokens,
                        float softmax_scale, int mask_mode, int64_t q_pos0,
                        int64_t chunk_tokens, void* out, int64_t out_sb, int64_t out_st,
                        int64_t out_sh, const float* rope_hw, int grid_h, int grid_w,
                        const float* q_xform_t, const float* q_xform_s, const float* out_xform,
                        int n_qframes, skv_stream_t stream);

/*
 * Commit-path fusion: the reference normalises K and Q with WanRMSNorm over each token's full
 * H x D row before the cache write and the attention (q = norm_q(q(x)), k = norm_k(k(x)),
 * causal_model.py:908-910; WanRMSNorm model.py:69-84: x * rsqrt(mean(x²) + eps) * weight).
 * Here the statistic is one small pass and the scaling is folded into the append (K) and into
 * the attention kernel's Q load, so the normalised K/Q never round-trip through HBM.
 *
 * skv_rms_rows — inv_rms[b * rows + t] = 1 / sqrt(mean over (h, d) of x[b][t][h][d]² + eps)
 * (fp32) for a token-major [batch][rows][heads][head_dim] tensor (bf16 or f32).
 */
int skv_rms_rows(const void* x, int dtype, int64_t sb, int64_t st, int64_t sh, int batch,
                 int rows, int heads, int head_dim, float eps, float* inv_rms /* device */,
                 skv_stream_t stream);

/*
 * Extended append: every option of skv_append / skv_append_rope / skv_append_prope plus the
 * RMSNorm of K.  Optional members are NULL / 0 when unused.
 *   k_inv_rms, k_rms_stride_b, k_norm_weight: source token t of stream b is stored as
 *     k * k_inv_rms[b * k_rms_stride_b + t] * k_norm_weight[h * head_dim + c], evaluated in fp32
 *     and rounded once to the source dtype (the reference rounds its bf16 norm several times);
 *     the RoPE / PRoPE copies and fp8 codes derive from that rounded value.  V is not normalised.
 *   kr_pool, rope_hw, grid_h, grid_w: the RoPE copy of K (skv_append_rope).
 *   vx_pool, kv_xform: the PRoPE copies (skv_append_prope; kr_pool then receives K with RoPE and
 *     P⁻¹ on its spatial groups).
 *   kr_scale, vx_scale: fp8 pools only, the copies' own scales ([n_slots][batch][heads] float32,
 *     absmax / 448 of each written (slot, stream, head) of kr_pool / vx_pool).  A copy's codes
 *     are the e4m3 encoding of exactly the value a bf16 (f32 for f32 sources) copy would hold;
 *     fp8 copies need the workspace skv_append_workspace_size reports.
 */
typedef struct skv_append_desc {
  const void* k_new;
  const void* v_new;
  int src_dtype;
  int64_t src_sb, src_st, src_sh;
  int src_frame0;
  void* k_pool;
  void* v_pool;
  float* k_scale;
  float* v_scale;
  int pool_dtype;
  int n_slots;
  const int32_t* dst_slots; /* host */
  int n_frames, batch, heads, head_dim, frame_tokens;
  const float* k_inv_rms;
  int64_t k_rms_stride_b;
  const float* k_norm_weight;
  void* kr_pool;
  const float* rope_hw;
  int grid_h, grid_w;
  void* vx_pool;
  const float* kv_xform;
  void* workspace;         /* device, optional, 4-byte aligned (8 for the one-pass fp8 kernel) */
  int64_t workspace_bytes; /* its size; must cover skv_append_workspace_size */
  float* kr_scale;         /* fp8 pools with kr_pool */
  float* vx_scale;         /* fp8 pools with vx_pool */
} skv_append_desc;

int skv_append_ex(const skv_append_desc* desc, skv_stream_t stream);

/*
 * Workspace skv_append_ex would use for `desc` (0 when the launch needs none: bf16/f32 pools,
 * or an fp8 chunk with enough units to fill the chip); validates like skv_append_ex.  No
 * reference counterpart (the reference append, causal_model.py:2894-2914, is a slice copy).
 */
int skv_append_workspace_size(const skv_append_desc* desc, int64_t* bytes);

/*
 * Extended attention: every option of skv_attention / skv_attention_rope / skv_attention_prope
 * plus the RMSNorm of Q at load (q_inv_rms[b * q_rms_stride_b + row] * q_norm_weight[h *
 * head_dim + c], fp32, before RoPE/PRoPE; the fp8-pool kernel rounds the normalised Q to bf16
 * before quantising it, as the reference's bf16 norm output).  Optional members NULL / 0.
 * rope_t selects RoPE on load, q_xform_t (with q_xform_s, out_xform) RoPE + PRoPE.  On fp8
 * pools with frames of at least 64 tokens RoPE on load multiplies e4m3 codes: each query row
 * is rounded to bf16, its height/width pairs turned and rounded to bf16, and for every key frame
 * its temporal pairs turned by rope_t and rounded to bf16, then quantised with one row scale
 * max(|turned height/width values|, temporal pair norms) / 448 (no code clips); shorter frames
 * and PRoPE decode the fp8 tiles to bf16 and multiply in bf16.
 * frame_lens (mask NONE only) lets frames hold fewer than frame_tokens keys, so a window can
 * mix whole frames with spans of other lengths (the H3 prefix rows, memory_kv_attention.py).
 * Segments (n_segments > 0, up to SKV_MAX_SEGMENTS; bf16 pools, bf16 or f32 queries, mask NONE,
 * no RoPE / PRoPE): the queries are n_segments consecutive row ranges of seg_rows[s] rows
 * (summing to q_len), and segment s attends only its own seg_frames[s] consecutive entries of
 * frame_slots / frame_lens (the lists of all segments end to end, summing to n_frames), in one
 * launch: the teacher-forcing block mask (causal_model.py:337-471) and the H3 segment layouts
 * (sgf_attention.py:236-258, memory_kv_attention.py:39-140) are such lists.
 */
typedef struct skv_attention_desc {
  const void* q;
  int q_dtype;
  int64_t q_sb, q_st, q_sh;
  const void* k_pool;
  const void* v_pool;
  const float* k_scale;
  const float* v_scale;
  int pool_dtype;
  int n_slots;
  const int32_t* frame_slots; /* host */
  int n_frames, batch, heads, head_dim, q_len, frame_tokens;
  float softmax_scale;
  int mask_mode;
  int64_t q_pos0, chunk_tokens;
  void* out;
  int64_t out_sb, out_st, out_sh;
  const float* q_inv_rms;
  int64_t q_rms_stride_b;
  const float* q_norm_weight;
  const float* rope_hw;
  int grid_h, grid_w;
  const float* rope_t;
  int n_qframes;
  const float* q_xform_t;
  const float* q_xform_s;
  const float* out_xform;
  const int32_t* frame_lens; /* host, optional: valid keys of each listed frame (1..frame_tokens;
                                keys past it are masked), for spans that are not whole frames */
  void* workspace;            /* device, optional, 16-byte aligned: enables the balanced key split */
  int64_t workspace_bytes;    /* its size; must cover skv_attention_plan's workspace_bytes */
  const int32_t* seg_rows;    /* host, n_segments entries: query rows of each segment */
  const int32_t* seg_frames;  /* host, n_segments entries: frame-list entries of each segment */
  int n_segments;             /* 0: one segment (every query over the whole frame list) */
} skv_attention_desc;

int skv_attention_ex(const skv_attention_desc* desc, skv_stream_t stream);

/*
 * The launch skv_attention_ex would make for `desc`, without launching (validates the same way
 * and returns the same status).  workspace_bytes > 0 means the balanced key split pays for this
 * shape and needs that much workspace; `split` says whether `desc` as given takes it (it does
 * exactly when desc->workspace is set and large enough).  No reference counterpart: the
 * reference attention (attention.py:141-188) has no launch choices to report.
 */
typedef struct skv_launch_plan {
  int waves_per_group;     /* 8 (256 queries per workgroup) or 4 (128) */
  int split;               /* 0: none; 1: balanced key split of every query tile over one
                              workgroup per CU + merge kernel; 2: the grid's full rounds run
                              unsplit and only the last, partly filled round's query tiles
                              are split over the CUs (+ merge kernel) */
  int n_workgroups;        /* workgroups of the attention kernel launches (both, for split 2) */
  int n_qtiles;            /* query tiles (over all batches and heads) */
  int64_t workspace_bytes; /* workspace the split needs; 0 when it does not pay */
  int key_tiles;           /* 64-key tiles per query tile over the whole window: n_frames x
                              ceil(T / 64), or ceil(n_frames x T / 64) when the bf16 / f16
                              kernel packs tiles across frame boundaries (whole frames, T a
                              multiple of 8 but not of 64, no RoPE): no padding keys computed */
} skv_launch_plan;

int skv_attention_plan(const skv_attention_desc* desc, skv_launch_plan* plan);

/*
 * H3 transforms (MiniMax-H3 backend).  H3's attention segments take rotate-half MM-RoPE on head
 * channels [0, 96) and its camera PRoPE on channels [96, 128) (eight 4-vectors per row, each
 * multiplied by the row's 4x4 matrix) before attention, and the output matrix on the attention
 * output's channels [96, 128) after it (sgf_attention.py:192-203, :580-659;
 * torch_prope.py:187-241).
 *
 * skv_h3_rope_prope — one pass over a [batch][rows][heads][128] bf16 tensor (any strides with
 * unit channel stride), replacing fused_prope.py:196-255 (rope_prope, the SGF rotary + camera
 * projection) and, with cos = sin = NULL, fused_prope.py:30-93 (prope_project):
 *   channels [0, 48) and [48, 96), x1 and x2, with c = bf16(cos[t]), s = bf16(sin[t]):
 *     y1 = bf16(bf16(x1 c1) + bf16(-x2 s1)),  y2 = bf16(bf16(x2 c2) + bf16(x1 s2));
 *   channels [96, 128), 4-vector v of row t: y_i = bf16(((M_i0 v_0 + M_i1 v_1) + M_i2 v_2)
 *     + M_i3 v_3) in fp32 with M = matrix[b][t] rounded to bf16 (products of bf16 values are
 *     exact in fp32, so this is the reference kernel's expression, bit for bit).
 * cos / sin: [rows][96] (row stride table_stride elements), bf16 or f32, or both NULL to copy
 * channels [0, 96).  matrix: [batch or 1][rows][4][4], bf16 or f32 (matrix_sb = 0 broadcasts
 * one set over the batch), or NULL to copy channels [96, 128).  out may be x itself (every
 * row is read before any of it is written) but must not otherwise overlap it.
 */
typedef struct skv_h3_xform_desc {
  const void* x;
  int64_t x_sb, x_st, x_sh;
  void* out;
  int64_t out_sb, out_st, out_sh;
  int batch, rows, heads, head_dim;
  const void* cos;
  const void* sin;
  int table_dtype;
  int64_t table_stride;
  const void* matrix;
  int matrix_dtype;
  int64_t matrix_sb, matrix_st;
} skv_h3_xform_desc;

int skv_h3_rope_prope(const skv_h3_xform_desc* desc, skv_stream_t stream);

/*
 * skv_attention_ex_noalloc — skv_attention_ex that allocates nothing and takes no workspace:
 * the balanced key split keeps its partial results in a static device array of
 * SKV_NOALLOC_SCRATCH_BYTES per GPU (2 records x 256 rows x 130 floats for each of up to 256
 * CUs), held by every GPU that calls it until the process ends.  desc->workspace must be NULL
 * and workspace_bytes 0; a launch whose split would need more scratch (a device with more than
 * 256 CUs) returns SKV_E_UNSUPPORTED.  Results equal skv_attention_ex's with a workspace.  All
 * calls on one GPU share its array, so calls that overlap on one GPU (different streams) race;
 * calls on one stream are ordered and safe.  No counterpart in the reference: it exists for
 * callers that cannot allocate device memory (code under HIP graph capture, serving loops that
 * forbid allocation).
 */
#define SKV_NOALLOC_SCRATCH_BYTES 68157440
int skv_attention_ex_noalloc(const skv_attention_desc* desc, skv_stream_t stream);

/*
 * skv_noalloc_init — set-up of skv_attention_ex_noalloc on the current device: looks up the
 * device address of that device's scratch array (loading the code object that holds it).  Call
 * it once per device, with the device current, before the first skv_attention_ex_noalloc made
 * under HIP graph capture: a captured call whose device is not set up returns SKV_E_UNSUPPORTED
 * instead of loading a module mid-capture.  Outside capture the entry point sets itself up on
 * first use.  Idempotent and thread-safe; allocates nothing beyond the static array.  No
 * counterpart in the reference (see skv_attention_ex_noalloc).
 */
int skv_noalloc_init(void);

#ifdef __cplusplus
}
#endif

#endif /* SOLARKV_H */
