/*
 * qvl_vision.h — C ABI of the MI355X (gfx950) Qwen3-VL vision-tower library (libqvl.so).
 *
 * Drop-in replacement for the reference's `Qwen3VLModel.encode_vision` hot path
 * (/root/reference/model.py:940-944 -> Qwen3VisionTransformer.__call__, model.py:801-851).
 * Each entry replaces one reference function; the citation is on each declaration.
 *
 * Conventions
 *   - Plain pointers and sizes only. Device pointers are marked `d_`, host pointers `h_`.
 *   - Every device entry is asynchronous on the caller's `stream` (a hipStream_t; NULL = the
 *     default stream) and never allocates: scratch comes in through `workspace`.
 *   - Return 0 (QVL_OK) or a negative QVL_ERR_* code; `qvl_last_error()` returns a message for
 *     the last failure on the calling thread. The only other state is thread-local
 *     (qvl_set_gemm_plan) or a write-once per-device cache (compute-unit counts, kernel
 *     attributes set once per process): entries are re-entrant and may be called concurrently
 *     from several host threads on different streams. One exception:
 *     qvl_attention_headmajor_split_noalloc keeps its partial outputs in one file-scope device
 *     array per GPU (no workspace argument), so calls of it that overlap on one GPU race.
 *   - Activations are row-major [tokens, features]. "Packed" dense weights are [n_out, k_in]
 *     row-major (the transpose of the reference's Flax kernel [in, out], model.py:1152-1153),
 *     with n_out and k_in zero-padded to multiples of 64; biases and LayerNorm affine
 *     parameters are float32 vectors (holding bf16-representable values in the bf16 mode).
 *   - Token order is the reference's 2x2 merge-block order (sample.py:112-119).
 *   - dtype: QVL_DTYPE_BF16 (bf16 storage and MFMA, fp32 accumulation / softmax / LayerNorm
 *     statistics) or QVL_DTYPE_F32 (the reference's default dtype: fp32 storage and arithmetic,
 *     fp32 MFMA); entries that exist for one of them only say so.
 */
#ifndef QVL_VISION_H
#define QVL_VISION_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define QVL_OK 0
#define QVL_ERR_INVALID_ARG (-1)   /* bad shape / pointer / grid (e.g. odd h or w) */
#define QVL_ERR_UNSUPPORTED (-2)   /* a shape or dtype this build has no kernel for */
#define QVL_ERR_MISALIGNED (-3)    /* a pointer or leading dimension is not 16-byte aligned */
#define QVL_ERR_WORKSPACE (-4)     /* workspace too small */
#define QVL_ERR_LAUNCH (-5)        /* a HIP launch failed */

#define QVL_DTYPE_F32 0
#define QVL_DTYPE_BF16 1

/* Epilogues of qvl_dense (all accumulate in fp32 and round once to the output dtype). */
#define QVL_EPI_BIAS 0            /* y = x W^T + b                         (nn.Dense)          */
#define QVL_EPI_BIAS_GELU 1       /* y = gelu_tanh(x W^T + b)              (Dense -> jax.nn.gelu) */
#define QVL_EPI_BIAS_RESIDUAL 2   /* y = x W^T + b + r   (r may alias y)   (Dense -> residual add) */

const char* qvl_last_error(void);
const char* qvl_status_string(int status);
int qvl_version(void);

/* ------------------------------------------------------------------------------------------ */
/* Host-side integer metadata, built once per grid_thw.                                        */
/* ------------------------------------------------------------------------------------------ */

/* Token and segment counts of a grid: n_tokens = sum t*h*w, n_segments = sum t.
 * Replaces the shape arithmetic of model.py:825-834. Rejects h or w not divisible by `merge`. */
int qvl_grid_counts(const int32_t* h_grid_thw, int64_t n_grids, int32_t merge,
                    int64_t* n_tokens, int64_t* n_segments);

/* Integer metadata of the tower, bit-exact with the reference:
 *   h_cu_seqlens [n_segments+1] int32  model.py:831-834 (one segment per frame)
 *   h_pos_hw     [n_tokens, 2]  int32  model.py:686-693 ((h, w) rotary ids, merge-block order)
 *   h_tap_idx    [4, n_tokens]  int32  model.py:713-739, 761-764 (bilinear taps into the
 *   h_tap_w      [4, n_tokens]  f32    learned table, incl. the jnp.repeat frame quirk);
 *                                      weights rounded to bf16 when dtype == QVL_DTYPE_BF16
 *                                      (model.py:749 casts them to the tower dtype).
 * Any output pointer may be NULL to skip it. */
int qvl_vision_metadata(const int32_t* h_grid_thw, int64_t n_grids, int32_t merge,
                        int32_t num_position_embeddings, int32_t dtype,
                        int32_t* h_cu_seqlens, int32_t* h_pos_hw, int32_t* h_tap_idx, float* h_tap_w);

/* Attention work list for qvl_vision_attention / qvl_attention_headmajor / qvl_encode_vision:
 * one int32 quadruple (segment start, segment end, first query, head) per query tile of the
 * kernel's tile height and per head. Replaces the per-segment Python loop of model.py:585-598.
 * Layout: (segment, head) groups, longest segment first, are dealt to 8 queues (one per XCD)
 * by least accumulated work (query tiles x keys); item k is entry k / 8 of queue k % 8, the
 * XCD that runs workgroup k, so a group's K/V stay in one L2. Short queues are padded with
 * empty items (start == end). With h_items == NULL only *n_items is written. */
int qvl_attention_worklist(const int32_t* h_cu_seqlens, int64_t n_segments, int32_t num_heads,
                           int32_t* h_items, int64_t capacity, int64_t* n_items);

/* The same work list balanced for the last round of workgroup slots (modelled on the bf16
 * kernels, head_dim 64 or 72; `n_cus` compute units, 4 or 3 workgroups each; the fp32 kernel runs
 * the same lists): the items that would run in the last,
 * partial round leave the list (their entries become empty items) and are appended as up to 8
 * parts each that split their key tiles (head field: head | part << 12 | parts << 20). Items
 * [0, *n_whole) are whole, [*n_whole, *n_items) parts, in item order. Same call convention as
 * qvl_attention_worklist. The per-segment loop of model.py:585-598, scheduled for one GPU. */
int qvl_attention_worklist_split(const int32_t* h_cu_seqlens, int64_t n_segments, int32_t num_heads,
                                 int32_t head_dim, int32_t n_cus, int32_t* h_items, int64_t capacity,
                                 int64_t* n_items, int64_t* n_whole);

/* Rotary inverse frequencies theta^(-2j/(head_dim/2)), j < head_dim/4, float32
 * (VisionRotaryEmbedding, model.py:540-546 with dim = head_dim/2, model.py:672). */
int qvl_rotary_inv_freq(int32_t head_dim, float theta, float* h_inv_freq);

/* ------------------------------------------------------------------------------------------ */
/* Device stages.                                                                              */
/* ------------------------------------------------------------------------------------------ */

/* Pack a reference Flax kernel [k_in, n_out] (float32, row-major) into the GEMM layout
 * [n_pad, k_pad] of `dtype` (n_pad, k_pad = round-up to 64, zero-filled).
 * Load-time counterpart of model.py:1152-1153 (HF weight.T) + the Dense promotion to dtype. */
int qvl_pack_dense_weight(void* stream, int32_t dtype, const float* d_kernel, int64_t k_in,
                          int64_t n_out, void* d_packed);

/* Cast float32 -> dtype (bf16 rounds to nearest even). Replaces `x.astype(dtype)` (model.py:556). */
int qvl_cast(void* stream, int32_t dtype, const float* d_x, void* d_y, int64_t n);

/* y[M, N] = epilogue(x[M, K] . W[N, K]^T + bias)  — nn.Dense call sites model.py:556, 570, 601,
 * 611-613, 655-656 with their following activation / residual add fused in.
 * K must be a multiple of 64 (packed weights are zero-padded); lda/ldc/ldr in elements. */
int qvl_dense(void* stream, int32_t dtype, int32_t epilogue, const void* d_x, int64_t lda,
              const void* d_w, const float* d_bias, const void* d_residual, int64_t ldr,
              void* d_y, int64_t ldc, int64_t m, int64_t n, int64_t k);

/* qvl_dense with a workspace for split-K: bf16, when the tiles do not fill whole rounds of the
 * GPU's compute units, the last round's tiles are split along K; fp32, when the 128 x 128 tiles
 * fill at most half of the workgroup slots (two per compute unit), every tile is split along K
 * into up to 8 parts. The parts' fp32 partials go to `d_workspace` and a second kernel sums them
 * (in part order) before the epilogue: same results up to fp32 summation order. Without enough
 * workspace it behaves exactly like qvl_dense.
 * qvl_dense_workspace_size gives the bytes that always suffice on the current device. */
int qvl_dense_workspace_size(size_t* bytes);
int qvl_dense_ws(void* stream, int32_t dtype, int32_t epilogue, const void* d_x, int64_t lda,
                 const void* d_w, const float* d_bias, const void* d_residual, int64_t ldr,
                 void* d_y, int64_t ldc, int64_t m, int64_t n, int64_t k,
                 void* d_workspace, size_t workspace_bytes);

/* Tile-plan override for the bf16 GEMMs (qvl_dense / qvl_dense_ws / qvl_dense_qkv_rotary and the
 * GEMMs inside qvl_encode_vision) launched afterwards FROM THE CALLING THREAD ONLY (thread-local;
 * other threads keep the cost model's choice). For tests and tuning sweeps, not needed by callers:
 *   tile       0 = cost model (default), 1 = 288x256, 2 = 256x256, 3 = 256x128, 4 = 288x128,
 *                5 = row split (the rows of whole rounds of 288x256 tiles, then the rest as
 *                256x128 tiles in a second launch; 288x256 where no such split exists),
 *                6 = 128x128 tiles (chosen by the default plan on small grids with K <= 1536),
 *                7 = 64x192 tiles (the head_dim-64 rotary qkv GEMM only: its default where one
 *                round of them fits the compute units), 8 = 64x128 tiles (the patch embed's
 *                default on small grids)
 *                (the head_dim-64 rotary qkv epilogue takes 1-3 and 5-8 and maps 4 to 3; for the
 *                head_dim-72 one, 0 = whole rounds of 256x288 tiles and the rest in 128x288
 *                tiles where that fits one round (64x288 where those fill at most half of it),
 *                1 = 256x288 tiles only, 2 = that row split wherever there are two 256-row
 *                tiles, 3 = the same with the rest in 64x288 tiles);
 *   split_mode 0 = cost model decides the tail split-K, 1 = force it, -1 = forbid it;
 *   group_n    column tiles per panel of the tile order, 0 = default (4).
 * (0, 0, 0) restores the defaults. No counterpart in the reference (it has no tile plans). */
int qvl_set_gemm_plan(int32_t tile, int32_t split_mode, int32_t group_n);

/* Key-group override for the head_dim-64 bf16 attention launched afterwards FROM THE CALLING THREAD
 * ONLY (thread-local), for tests and tuning: 0 = the default rule (two groups of 4 waves per work
 * item, each taking half of the item's key tiles and combined in LDS, where the items number at
 * most 2x the compute units; else one group), 1 = one group, 2 = two groups. Outputs of 1 and 2 differ
 * only in fp32 summation order. No counterpart in the reference. */
int qvl_set_attention_plan(int32_t key_groups);

/* LayerNorm over the last axis: fp32 mean / biased variance / rsqrt(var + eps), affine, cast
 * back (model.py:375-388). cols must be a multiple of 8 and <= 8192. bf16 or fp32. */
int qvl_layer_norm(void* stream, int32_t dtype, const void* d_x, int64_t ldx, const float* d_gamma,
                   const float* d_beta, void* d_y, int64_t ldy, int64_t rows, int64_t cols, float eps);

/* Bilinear pos-embed: y[n, :] = sum_j w[j, n] * table[idx[j, n], :] (model.py:751-764).
 * `d_table` is [num_position_embeddings, dim] in dtype. */
int qvl_pos_embed(void* stream, int32_t dtype, const void* d_table, const int32_t* d_tap_idx,
                  const float* d_tap_w, void* d_y, int64_t n_tokens, int64_t dim);

/* Rotary table cs[n, j] = (cos, sin)(pos * inv_freq) as float2 [n_tokens, head_dim/2], with
 * pos = pos_hw[n, 0] for j < head_dim/4 else pos_hw[n, 1] (model.py:694-698, 821-823);
 * values rounded to bf16 when dtype == QVL_DTYPE_BF16 (`.astype(self.dtype)`, model.py:823). */
int qvl_rotary_table(void* stream, int32_t dtype, const int32_t* d_pos_hw, int64_t n_tokens,
                     int32_t head_dim, float theta, void* d_cos_sin);

/* Packed varlen vision attention with 2D rotary (model.py:569-600 between the qkv and proj
 * Dense): q/k/v are [n_tokens, num_heads*head_dim] views (row stride ld_qkv elements, e.g. the
 * three column blocks of the qkv Dense output), rotated in-kernel with `d_cos_sin`
 * (qvl_rotary_table), then softmax(q k^T / sqrt(head_dim)) v per cu_seqlens segment
 * (block-diagonal, non-causal, fp32 online softmax). Output [n_tokens, num_heads*head_dim]
 * row stride ld_out. `d_tiles` / `n_tiles` are the qvl_attention_worklist items (device copy)
 * and their count.
 * Workspace: qvl_vision_attention_workspace_size(). head_dim in {64, 72, 80}. */
int qvl_vision_attention_workspace_size(int32_t dtype, int64_t n_tokens, int32_t num_heads, int32_t head_dim,
                                        size_t* bytes);
int qvl_vision_attention(void* stream, int32_t dtype, const void* d_q, const void* d_k,
                         const void* d_v, int64_t ld_qkv, const void* d_cos_sin,
                         const int32_t* d_tiles, int64_t n_tiles, void* d_out, int64_t ld_out,
                         int64_t n_tokens, int32_t num_heads, int32_t head_dim,
                         void* d_workspace, size_t workspace_bytes);

/* Fused qkv Dense + rotary (model.py:570-582): one GEMM x[N, D] . Wqkv[3D, D]^T + b whose
 * epilogue applies the 2D rotary to q and k with `d_cos_sin` (qvl_rotary_table of this head_dim)
 * and writes the head-major operands of qvl_attention_headmajor, Np = n_tokens rounded up to 64,
 * rows / positions [n_tokens, Np) zeroed:
 *   head_dim 64 (D a multiple of 128): q (scaled by head_dim^-0.5 * log2(e)) and k as
 *     [H][Np][64], v transposed as [H][64][Np] (keys at their vt_pos positions);
 *   head_dim 72 (num_heads a multiple of 4): q (scaled) and k as [H][Np][88] with dims 72..87
 *     zero, v transposed as [H][72][Np].
 * Every rounding is the reference's (bf16 Dense output, bias add, each rotary product and sum).
 * bf16 only (the fp32 tower runs qvl_dense and qvl_vision_attention). The optional workspace
 * (qvl_dense_workspace_size bytes, may be NULL) enables tail split-K for head_dim 64 as in
 * qvl_dense_ws. */
int qvl_dense_qkv_rotary(void* stream, int32_t dtype, const void* d_x, int64_t lda, const void* d_w,
                         const float* d_bias, const void* d_cos_sin, void* d_q, void* d_k, void* d_vt,
                         int64_t n_tokens, int64_t hidden, int32_t num_heads,
                         void* d_workspace, size_t workspace_bytes);

/* Per-position rotary table for qvl_dense_qkv_rotary_pos: table[p][j] = bf16(cos) | bf16(sin) << 16
 * of p * inv_freq[j] for p < n_positions, j < head_dim/4 (uint32 [n_positions][head_dim/4]): the
 * (cos, sin) qvl_rotary_table gives a token at rotary id p, bit for bit (model.py:540-546,
 * 694-698, 821-823 with the angle's two axes sharing one table). */
int qvl_rotary_pos_table(void* stream, int32_t head_dim, float theta, int32_t n_positions, uint32_t* d_table);

/* qvl_dense_qkv_rotary with (cos, sin) looked up by each token's rotary (h, w) ids (`d_pos_hw`
 * [n_tokens][2] of qvl_vision_metadata, every id < n_positions) in a qvl_rotary_pos_table table,
 * which the kernel keeps in LDS instead of reading a per-token table: same outputs bit for bit.
 * n_positions * head_dim/4 * 4 bytes must fit 16384 (head_dim 64) or 12288 (head_dim 72) bytes. */
int qvl_dense_qkv_rotary_pos(void* stream, int32_t dtype, const void* d_x, int64_t lda, const void* d_w,
                             const float* d_bias, const int32_t* d_pos_hw, const uint32_t* d_table,
                             int32_t n_positions, void* d_q, void* d_k, void* d_vt, int64_t n_tokens,
                             int64_t hidden, int32_t num_heads, void* d_workspace, size_t workspace_bytes);

/* LayerNorm folded into the Dense that consumes it (LayerNorm model.py:375-388, feeding the qkv
 * Dense at 570 via norm1 (628), linear_fc1 at 611 via norm2 (629), and a deepstack merger's
 * linear_fc1 at 651-655 via its post-shuffle norm). With xn = (x - mean) * rstd * gamma + beta:
 *   xn . W[n] = rstd * (x . W'[n]) - rstd * mean * c[n] + d[n],
 *   W'[n][k] = bf16(gamma[k] * W[n][k]),  c[n] = sum_k W'[n][k],  d[n] = sum_k beta[k] * W[n][k],
 * so the Dense runs on the un-normalised rows x with the folded kernel W', and the per-row
 * (mean, rstd) and per-feature (c, d) are applied to the fp32 accumulator before the bias and the
 * rest of the epilogue (the bf16 rounding of the product then happens where the reference rounds
 * its Dense output; the reference's rounding of xn to bf16 is replaced by the rounding of W').
 * bf16 only. */

/* (mean, rsqrt(var + eps)) of each row of x [rows, cols] (bf16, row stride ldx), two-pass fp32 as in
 * qvl_layer_norm: d_stats [rows][2] fp32. (model.py:384-386) */
int qvl_row_stats(void* stream, int32_t dtype, const void* d_x, int64_t ldx, int64_t rows, int64_t cols,
                  float eps, float* d_stats);

/* W' and (c, d) from a qvl_pack_dense_weight kernel: d_w and d_out_w packed [round_up(n_out, 64), k_in]
 * (k_in a multiple of 64), d_out_cd [round_up(n_out, 64)][2] fp32; padding rows give zeros.
 * d_gamma / d_beta: the LayerNorm's [k_in] affine (bf16-representable fp32 values). */
int qvl_fold_ln_weight(void* stream, int32_t dtype, const void* d_w, int64_t k_in, int64_t n_out,
                       const float* d_gamma, const float* d_beta, void* d_out_w, float* d_out_cd);

/* qvl_dense_ws on the un-normalised rows with a folded LayerNorm (QVL_EPI_BIAS or
 * QVL_EPI_BIAS_GELU): d_w = W', d_cd = (c, d) of qvl_fold_ln_weight, d_stats = qvl_row_stats of x. */
int qvl_dense_ln_ws(void* stream, int32_t dtype, int32_t epilogue, const void* d_x, int64_t lda,
                    const void* d_w, const float* d_cd, const float* d_stats, const float* d_bias,
                    void* d_y, int64_t ldc, int64_t m, int64_t n, int64_t k,
                    void* d_workspace, size_t workspace_bytes);

/* qvl_dense_qkv_rotary (d_cos_sin != NULL, d_pos_hw / d_table NULL) or qvl_dense_qkv_rotary_pos
 * (d_cos_sin NULL) with norm1 folded in: x un-normalised, d_w = W', d_cd, d_stats as above. */
int qvl_dense_qkv_rotary_ln(void* stream, int32_t dtype, const void* d_x, int64_t lda, const void* d_w,
                            const float* d_cd, const float* d_stats, const float* d_bias,
                            const void* d_cos_sin, const int32_t* d_pos_hw, const uint32_t* d_table,
                            int32_t n_positions, void* d_q, void* d_k, void* d_vt, int64_t n_tokens,
                            int64_t hidden, int32_t num_heads, void* d_workspace, size_t workspace_bytes);

/* The row statistics of a folded LayerNorm produced by the Dense that writes its input: the
 * residual Dense (x + proj / fc2, model.py:628-629; the patch embed + pos-embed, 802-806) also
 * writes, per output row m and 128-column group g, d_parts[m][g] = (sum_j y, sum_j (y - mean_g)^2)
 * over the group's bf16 outputs y (n % 128 == 0, ldc and ldr multiples of 8; d_parts
 * [m][n / 128][2] fp32). The folded Dense entries below combine a row's groups into its mean and
 * variance (Chan et al.'s pairwise update), which replaces the LayerNorm's statistics pass
 * (model.py:384-386): no LayerNorm and no statistics launch remain between the two GEMMs. bf16.
 * With a workspace the tail tiles may split along K (qvl_dense_ws); the split-K reduction then writes
 * their rows' partials. */
int qvl_dense_rowstats_ws(void* stream, int32_t dtype, const void* d_x, int64_t lda, const void* d_w,
                          const float* d_bias, const void* d_residual, int64_t ldr, void* d_y, int64_t ldc,
                          int64_t m, int64_t n, int64_t k, float* d_parts, void* d_workspace,
                          size_t workspace_bytes);

/* The patch embed with the learned pos-embed added in its epilogue (model.py:549-556, 751-764,
 * 802-806): y = bf16(bf16(bf16(x . W) + bias) + pos), where row m's pos is gathered from its 4
 * bilinear taps (d_tap_idx / d_tap_w [4][m], as qvl_vision_metadata writes them) over d_table
 * [*, n] in the arithmetic of qvl_pos_embed (each tap product and partial sum rounded to bf16), so
 * y equals qvl_pos_embed followed by the residual Dense bit for bit without the [m, n] pos-embed
 * buffer. d_parts non-NULL: also the row partials of qvl_dense_rowstats_ws (n % 128 == 0). bf16,
 * n and ldc multiples of 8; no split-K (the workspace is unused). */
int qvl_dense_pos_embed_ws(void* stream, int32_t dtype, const void* d_x, int64_t lda, const void* d_w,
                           const float* d_bias, const void* d_table, const int32_t* d_tap_idx, const float* d_tap_w,
                           void* d_y, int64_t ldc, int64_t m, int64_t n, int64_t k, float* d_parts,
                           void* d_workspace, size_t workspace_bytes);

/* qvl_dense_ln_ws with the row statistics given as qvl_dense_rowstats_ws partials of x: `groups`
 * 128-column groups per row (k == 128 * groups; a row of the deepstack mergers' [N/4, 4D] view is 4
 * token rows, i.e. 4 * D / 128 groups), eps the LayerNorm's (model.py:375-388). */
int qvl_dense_ln_parts_ws(void* stream, int32_t dtype, int32_t epilogue, const void* d_x, int64_t lda,
                          const void* d_w, const float* d_cd, const float* d_parts, int32_t groups, float eps,
                          const float* d_bias, void* d_y, int64_t ldc, int64_t m, int64_t n, int64_t k,
                          void* d_workspace, size_t workspace_bytes);

/* qvl_dense_qkv_rotary_ln with the row statistics as qvl_dense_rowstats_ws partials (hidden == 128 *
 * groups), model.py:628 + 570-582. */
int qvl_dense_qkv_rotary_ln_parts(void* stream, int32_t dtype, const void* d_x, int64_t lda, const void* d_w,
                                  const float* d_cd, const float* d_parts, int32_t groups, float eps,
                                  const float* d_bias, const void* d_cos_sin, const int32_t* d_pos_hw,
                                  const uint32_t* d_table, int32_t n_positions, void* d_q, void* d_k, void* d_vt,
                                  int64_t n_tokens, int64_t hidden, int32_t num_heads, void* d_workspace,
                                  size_t workspace_bytes);

/* The varlen attention kernel alone, on head-major operands (model.py:585-600):
 * out[n, h*head_dim + d] for every n inside a segment of `d_tiles`. Layout for head_dim 64: the
 * one qvl_dense_qkv_rotary writes; for head_dim 72 or 80: q, k [H][Np][88] (dims head_dim..87
 * zero) and v^T [H][head_dim][Np], keys at the same quad-swapped positions. fp32: q, k
 * [H][Np][head_dim], v^T [H][32*ceil(head_dim/32)][Np] (extra rows zero), keys in order. */
int qvl_attention_headmajor(void* stream, int32_t dtype, const void* d_q, const void* d_k, const void* d_vt,
                            const int32_t* d_tiles, int64_t n_tiles, int64_t n_tokens, int32_t num_heads,
                            int32_t head_dim, void* d_out, int64_t ld_out);

/* qvl_attention_headmajor on a qvl_attention_worklist_split list (bf16 or fp32, in
 * qvl_attention_headmajor's layouts): the parts write their unnormalised outputs and softmax state
 * to the workspace (qvl_attention_split_workspace_size(head_dim, n_tiles, n_whole) bytes) and a
 * combine kernel writes those items' rows (model.py:585-600). */
int qvl_attention_split_workspace_size(int32_t head_dim, int64_t n_tiles, int64_t n_whole, size_t* bytes);
int qvl_attention_headmajor_split(void* stream, int32_t dtype, const void* d_q, const void* d_k,
                                  const void* d_vt, const int32_t* d_tiles, int64_t n_tiles, int64_t n_whole,
                                  int64_t n_tokens, int32_t num_heads, int32_t head_dim, void* d_out,
                                  int64_t ld_out, void* d_workspace, size_t workspace_bytes);

/* qvl_attention_headmajor_split without a workspace argument: the parts' partial outputs go to a
 * scratch array inside the library (a static device array of qvl_noalloc_scratch_bytes() = 40 MiB,
 * one per GPU, held until the process ends), so the call allocates nothing and needs no caller
 * workspace. No counterpart in the reference: it exists for callers that cannot allocate device
 * memory (code under HIP graph capture, tight serving loops, harnesses that forbid hipMalloc).
 * A list whose parts need more than the scratch (qvl_attention_split_workspace_size) is refused
 * with QVL_ERR_WORKSPACE; every other check is qvl_attention_headmajor_split's. All calls on one
 * GPU share its scratch: calls that overlap in time on one GPU (several streams, or host threads)
 * race on it and must be serialised by the caller. Nothing in it needs clearing between calls
 * (each part writes every partial row the combine reads). */
size_t qvl_noalloc_scratch_bytes(void);
int qvl_attention_headmajor_split_noalloc(void* stream, int32_t dtype, const void* d_q, const void* d_k,
                                          const void* d_vt, const int32_t* d_tiles, int64_t n_tiles,
                                          int64_t n_whole, int64_t n_tokens, int32_t num_heads, int32_t head_dim,
                                          void* d_out, int64_t ld_out);

/* ------------------------------------------------------------------------------------------ */
/* Whole tower: Qwen3VisionTransformer.__call__ (model.py:801-851) / encode_vision (940-944).   */
/* ------------------------------------------------------------------------------------------ */

typedef struct qvl_vision_config {
  int32_t hidden_size;              /* D                                   */
  int32_t out_hidden_size;          /* merger output width                 */
  int32_t depth;
  int32_t num_heads;
  int32_t intermediate_size;        /* I (unpadded)                        */
  int32_t patch_volume;             /* C * Tp * P * P                      */
  int32_t spatial_merge_size;       /* must be 2                           */
  int32_t num_position_embeddings;  /* 0: no learned pos-embed (pos_table / taps unused)  */
  int32_t n_deepstack;
  int32_t deepstack_indexes[8];
  float ln_eps;                     /* 1e-6                                */
  float rope_theta;                 /* 10000                               */
  int32_t dtype;                    /* QVL_DTYPE_BF16 or QVL_DTYPE_F32     */
  int32_t use_window;               /* 1: window attention on the blocks not in fullatt_mask
                                       (model.py:808-850; fullatt_block_indexes != all)   */
  uint64_t fullatt_mask;            /* window mode: bit i = block i attends over the full
                                       cu_seqlens (depth <= 64)                          */
} qvl_vision_config;

/* A LayerNorm folded into the Dense after it (qvl_fold_ln_weight); w == NULL: not folded. */
typedef struct qvl_ln_fold {
  const void* w;                             /* packed W' [n_out_pad, k_in] bf16     */
  const float* cd;                           /* [n_out_pad][2] (c, d) fp32           */
} qvl_ln_fold;

typedef struct qvl_block_weights {           /* blocks_{i} (model.py:617-630)          */
  const float* norm1_w; const float* norm1_b;
  const float* norm2_w; const float* norm2_b;
  const void* qkv_w;  const float* qkv_b;    /* packed [3D, D]                        */
  const void* proj_w; const float* proj_b;   /* packed [D, D]                         */
  const void* fc1_w;  const float* fc1_b;    /* packed [I_pad, D]                     */
  const void* fc2_w;  const float* fc2_b;    /* packed [D, I_pad]                     */
  /* bf16 towers: norm1 folded into qkv and norm2 into fc1. When both are set the tower runs
   * qvl_row_stats + the folded GEMMs instead of the two qvl_layer_norm launches. */
  qvl_ln_fold qkv_ln, fc1_ln;
} qvl_block_weights;

typedef struct qvl_merger_weights {          /* merger / deepstack_mergers_{j} (633-656) */
  const float* norm_w; const float* norm_b;  /* [D] (main) or [4D] (deepstack)         */
  const void* fc1_w; const float* fc1_b;     /* packed [4D, 4D]                        */
  const void* fc2_w; const float* fc2_b;     /* packed [Dout_pad, 4D]                  */
  /* deepstack mergers in bf16: the post-shuffle norm folded into fc1 (the main merger's norm
   * acts per token on a row of 4 tokens, which one accumulator cannot take: never folded) */
  qvl_ln_fold fc1_ln;
} qvl_merger_weights;

typedef struct qvl_vision_weights {
  const void* patch_w; const float* patch_b; /* packed [D, patch_volume] (model.py:1136-1139) */
  const void* pos_table;                     /* [num_position_embeddings, D] in dtype         */
  const qvl_block_weights* blocks;           /* HOST array [depth]                             */
  qvl_merger_weights merger;
  const qvl_merger_weights* deepstack;       /* HOST array [n_deepstack]                       */
} qvl_vision_weights;

/* Window-attention metadata (model.py:769-799 `_get_window_index`, host side, bit-exact):
 * window_index [n_tokens/merge^2]: the merge group at each position of the window order (windows
 * of vit = window_size/merge/patch_size groups square, row-major per frame, groups row-major inside
 * a window, grids padded to whole windows and the padding skipped); cu_window: window boundaries
 * in tokens with consecutive duplicates removed, *n_cu_window entries (pass cu_window = NULL to
 * query the count). cu_full [n_grids + 1]: the full-attention cu_seqlens the reference uses in the
 * window path (model.py:828-830: cumsum of t*h*w*merge^2 per image), each clamped to n_tokens as
 * its q[start:end] slicing clamps it. Any output may be NULL. */
int qvl_window_metadata(const int32_t* h_grid_thw, int64_t n_grids, int32_t merge, int32_t patch_size,
                        int32_t window_size, int32_t* h_window_index, int32_t* h_cu_window, int64_t capacity,
                        int64_t* n_cu_window, int32_t* h_cu_full);

/* dst[r, :width] = src[idx[r / group] * group + r % group, :width], converted to dst_dtype (bf16
 * rounds to nearest even); n_rows (output rows) a multiple of group. The window path's merge-group
 * shuffle (model.py:809-812, group = merge^2) and unshuffle (845-848, group = 1). */
int qvl_gather_rows(void* stream, int32_t src_dtype, const void* d_src, int64_t ld_src, int32_t dst_dtype,
                    void* d_dst, int64_t ld_dst, const int32_t* d_idx, int64_t n_rows, int32_t group,
                    int64_t width);

/* Device metadata of one grid (qvl_vision_metadata / qvl_attention_worklist, copied to the GPU). */
typedef struct qvl_vision_metadata_dev {
  int64_t n_tokens;
  int64_t n_tiles;
  const int32_t* pos_hw;    /* [n_tokens, 2]  */
  const int32_t* tap_idx;   /* [4, n_tokens]  */
  const float* tap_w;       /* [4, n_tokens]  */
  const int32_t* tiles;     /* [n_tiles, 4]   */
  /* window mode only (else 0 / NULL): `tiles` are the worklist of cu_full, these of cu_window,
   * and pos_hw / tap_idx / tap_w are in window order (row r = token window_order[r]). */
  int64_t n_window_tiles;
  const int32_t* window_tiles;    /* [n_window_tiles, 4]                                     */
  const int32_t* window_index;    /* [n_tokens/4] merge group at each window-order position  */
  const int32_t* window_reverse;  /* [n_tokens/4] argsort(window_index)                      */
  /* optional (bf16 and fp32): a qvl_attention_worklist_split list of the full-attention
   * segments, used instead of `tiles` when split_tiles is not NULL. */
  int64_t n_split_tiles;
  int64_t n_split_whole;
  const int32_t* split_tiles;     /* [n_split_tiles, 4]                                      */
  /* optional: 1 + the largest rotary id in pos_hw (0 = unknown); lets the bf16 tower look
   * (cos, sin) up per position (qvl_dense_qkv_rotary_pos) */
  int64_t n_positions;
} qvl_vision_metadata_dev;

int qvl_encode_vision_workspace_size(const qvl_vision_config* cfg, int64_t n_tokens, size_t* bytes);

/* tokens [n_tokens/4, out_hidden_size] and deepstack[j] [n_tokens/4, out_hidden_size] in dtype
 * (the VisionEmbeddings pytree, model.py:27-31); `d_deepstack` is a HOST array of n_deepstack
 * device pointers. pixel_values: [n_tokens, patch_volume] float32 (model.py:556 input). */
int qvl_encode_vision(void* stream, const qvl_vision_config* cfg, const qvl_vision_weights* weights,
                      const qvl_vision_metadata_dev* meta, const float* d_pixel_values,
                      void* d_tokens, void* const* d_deepstack, void* d_workspace,
                      size_t workspace_bytes);

/* ------------------------------------------------------------------------------------------ */
/* The steps either side of the tower: patchify before it, decoder-side injection after it.    */
/* ------------------------------------------------------------------------------------------ */

/* On-device patchify: replaces the array part of `preprocess_image` (sample.py:86-121), i.e.
 * everything after PIL's convert("RGB") / resize. `d_frames` is uint8 [n_frames][height][width]
 * [channels] (HWC per frame, channels 3 or 4; a 4th channel is dropped like sample.py:74-75).
 * Writes pixel_values [gt*gh*gw, 3*Tp*P*P] (row stride ld_out elements) in dtype: value =
 * ((u8 / 255) - 0.5) / 0.5 computed in float32 exactly as sample.py:86-87 (bf16 output is that
 * value rounded to nearest even, i.e. `pixel_values.astype(bf16)` of model.py:556), frames padded
 * to a multiple of temporal_patch_size by repeating the last one (sample.py:93-98), rows in
 * merge-block order and columns (c, tp, ph, pw) (sample.py:112-119); gt = ceil(n_frames / Tp),
 * gh = height / P, gw = width / P. Errors like sample.py:104-110: height/width not divisible by
 * P, or gh/gw not divisible by merge_size -> QVL_ERR_INVALID_ARG. */
int qvl_patchify(void* stream, int32_t dtype, const uint8_t* d_frames, int64_t n_frames, int64_t height,
                 int64_t width, int32_t channels, int32_t patch_size, int32_t temporal_patch_size,
                 int32_t merge_size, void* d_out, int64_t ld_out);

/* Vision-token positions (model.py:927-931 `visual_mask` / `jnp.where(..., size=n, fill_value=-1)`,
 * also model.py:880-882): for each of `batch` rows of `d_tokens` [batch][seq_len] (int32), the
 * first n_rows indices s with tokens[s] == match, increasing, then -1; d_count[b] = the number of
 * matches (may exceed n_rows). A boolean mask works with tokens = mask as int32 and match = 1. */
int qvl_vision_positions(void* stream, const int32_t* d_tokens, int64_t batch, int64_t seq_len, int32_t match,
                         int64_t n_rows, int32_t* d_pos, int32_t* d_count);

#define QVL_SCATTER_SET 0   /* `_inject`: hidden[pos] = rows            (model.py:932-935) */
#define QVL_SCATTER_ADD 1   /* `_apply_deepstack`: hidden[pos] += rows  (model.py:880-886) */

/* hidden [batch][seq_len][dim] (hidden_dtype) at row d_pos[b][j] gets rows[b][j] (rows_dtype,
 * cast to hidden_dtype first, `feat.astype(h.dtype)`), for j < n_rows with 0 <= pos < seq_len
 * (a position past the row is dropped, as XLA drops out-of-bounds scatter updates); ADD rounds
 * hidden + row to hidden_dtype. `rows_batch_stride` (elements) is 0 to use one set of rows for
 * every batch row (VisionEmbeddings.with_batch_dim, model.py:47-63). `d_pos` / `d_count` come from
 * qvl_vision_positions. Where a row has fewer matches than n_rows, the reference's unfilled
 * updates all land on row 0 (a re-write of its old value after SET, a +0 after ADD); they are
 * applied in update order, as XLA's CPU scatter does. */
int qvl_scatter_vision_rows(void* stream, int32_t mode, int32_t hidden_dtype, void* d_hidden, int64_t batch,
                            int64_t seq_len, int64_t dim, int32_t rows_dtype, const void* d_rows,
                            int64_t rows_batch_stride, int64_t n_rows, const int32_t* d_pos,
                            const int32_t* d_count);

#ifdef __cplusplus
}
#endif
#endif /* QVL_VISION_H */
