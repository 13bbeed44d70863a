// Launchers of the gfx950 kernels (each .hip file defines its own), shared with the host entries.
#pragma once
#include <algorithm>

#include "qvl_common.h"
#include "qvl_host_common.h"

namespace qvl {

// kEpiBiasPosEmbed: the residual epilogue whose residual is the learned pos-embed, gathered per row from
// its bilinear taps (the patch embed of the tower, model.py:802-806).
enum : int { kEpiBias = 0, kEpiBiasGelu = 1, kEpiBiasResidual = 2, kEpiQkvRope = 3, kEpiQkvRope72 = 4,
             kEpiBiasPosEmbed = 5 };

struct GemmParams {
  const bf16* x; int64_t lda;
  const bf16* w;                 // [N, K] (ldw == K)
  const float* bias;             // [N]
  const bf16* res; int64_t ldr;  // residual, may alias y
  bf16* y; int64_t ldc;
  int M, N, K;
  // kEpiQkvRope: q/k written [H][Np][64] (rotated; q scaled by qscale), v written [H][64][Np].
  // kEpiQkvRope72: q/k written [H][Np][88] (dims 72..87 zero), v written [H][72][Np].
  bf16* q; bf16* k; bf16* vt;
  const f32x2* cs;               // [M, cs_half] (cos, sin), cs_half = head_dim / 2
  int cs_half;
  // Alternatively (rtab != NULL): cos / sin looked up by rotary position from a per-position
  // table rtab[P][head_dim / 4] of packed (bf16 cos | bf16 sin << 16), staged in LDS, with the
  // token's (h, w) ids from pos_hw [M][2].
  const int* pos_hw;
  const uint32_t* rtab;
  int rtab_pos;
  int Np, D;
  float qscale;
  // Tail split-K: fp32 partials workspace (NULL: no splitting) and its capacity in floats; the
  // launcher fills full_tiles / split.
  float* part;
  int64_t part_elems;
  int full_tiles, split;
  int group_n;                   // tile order: panels of group_n column tiles (set by the launcher)
  // Rows this launch covers: [row0, row1), row1 = 0 meaning max(M, Np) (zero-initialised params
  // cover every row). The head_dim-72 qkv plan runs its rows in two launches of different tile
  // heights; the outputs stay indexed by absolute row (no split-K tail with a row range).
  int row0, row1;
  // LayerNorm folded into this Dense (ln_stats != NULL): x holds the un-normalised rows, w the
  // folded kernel W' = bf16(gamma W), ln_stats[m] = (mean, rstd) of row m and ln_cd[n] = (c, d);
  // the accumulator becomes rstd * acc - rstd * mean * c + d before the epilogue.
  const f32x2* ln_stats;
  const f32x2* ln_cd;
  // ... or with the row statistics as per-128-column partials (ln_part != NULL instead of ln_stats):
  // ln_part[m * ln_groups + g] = (sum, sum of squared deviations from the group mean) of row m's
  // columns [128 g, 128 g + 128), K = 128 ln_groups, combined per row in the kernel (eps = ln_eps).
  const f32x2* ln_part;
  int ln_groups;
  float ln_eps;
  // Residual epilogue: also write those partials of the bf16 output rows (rs_part[m * N / 128 + g]),
  // the statistics of the LayerNorm that reads them next (N % 128 == 0, no split-K tail).
  f32x2* rs_part;
  // kEpiBiasPosEmbed: row m's residual is sum_j pe_w[j][m] * pe_table[pe_idx[j][m]][:] (j < 4, taps
  // [4][M], table rows of N bf16), in the pos-embed kernel's bf16 arithmetic (no split-K tail).
  const bf16* pe_table;
  const int* pe_idx;
  const float* pe_w;
};

// fp32 GEMM (qvl_f32.hip): w packed [n_rows_w][ldw] fp32 (ldw = k padded to 64), Kp = ldw.
struct GemmF32Params {
  const float* x; int64_t lda;
  const float* w; int64_t ldw; int64_t n_rows_w;
  const float* bias;
  const float* res; int64_t ldr;   // residual, may alias y
  float* y; int64_t ldc;
  int M, N, K, Kp;
  // Split-K (part != NULL, set by gemm_f32 when the tiles leave most workgroup slots idle): unit u
  // of the grid is K part u / tiles of tile u % tiles and stores its raw sums to
  // part[(u / tiles) * M * Npad + m * Npad + n] (Npad = N rounded up to the tile); a reduction
  // kernel sums the parts in order and applies the epilogue.
  float* part; int64_t part_elems;
  int split;
};

// Floats of split-K partial workspace that lets every GEMM of up to 256x256 tiles split its tail
// on a device with `cus` compute units (one tail unit per CU, at most one tile of partials each).
inline int64_t gemm_partials_elems(int cus) { return (int64_t)cus * 256 * 256; }
int gemm_device_cus();

// (work item head-field layout: qvl_host_common.h)
constexpr int kAttnBM = 128;   // queries per attention work item (bf16 and fp32 kernels)
__host__ __device__ constexpr int64_t attn_partial_floats(int hd) { return kAttnBM * (int64_t)(hd + 2); }   // per split slot

// Position of key m in the V^T layout the attention kernel reads: within each 16-key group
// (aligned to 16 in the token index) the middle two 4-key quads are swapped, so that the 8 keys a
// lane needs as the PV MFMA's k-slots are one contiguous 16-byte chunk.
__host__ __device__ __forceinline__ int vt_pos(int m) {
  const int q = (m >> 2) & 3;
  const int qs = (q == 1) ? 2 : (q == 2 ? 1 : q);
  return (m & ~15) | (qs << 2) | (m & 3);
}

int gemm_bf16(const GemmParams& p, int epi, hipStream_t stream);
// LDS bytes the qkv rotary epilogue can give to a per-position rotary table (head_dim 64 / 72),
// with a folded LayerNorm (ln: its (c, d) and row statistics take 4.3 KB of the 160 KB) or without.
__host__ __device__ constexpr int rope_table_lds_bytes(int hd, bool ln = false) {
  return hd == 64 ? (ln ? 12032 : 16384) : (ln ? 7936 : 12288);
}
int rotary_pos_table(int n_pos, int head_dim, const float* inv_freq, uint32_t* table, hipStream_t stream);
int gemm_set_plan(int tile, int split_mode, int group_n);
int attention_set_plan(int key_groups);
int attention_hd64(const bf16* Qb, const bf16* Kb, const bf16* Vtb, const int* d_tiles, int64_t n_tiles, int Np,
                   int H, bf16* out, int64_t ldo, hipStream_t stream, int64_t n_whole = -1, float* part = nullptr);
int attention_relayout_hd64(const bf16* q, const bf16* k, const bf16* v, int64_t ld, const f32x2* cs, int N, int Np,
                            int H, float qscale, bf16* Qo, bf16* Ko, bf16* Vto, hipStream_t stream);
int attention_general(const bf16* Qb, const bf16* Kb, const bf16* Vtb, const int* d_tiles, int64_t n_tiles, int Np,
                      int H, int hd, bf16* out, int64_t ldo, hipStream_t stream, int64_t n_whole = -1,
                      float* part = nullptr);
int attention_relayout_general(const bf16* q, const bf16* k, const bf16* v, int64_t ld, const f32x2* cs, int N, int Np,
                               int H, int hd, int HDP, int VROWS, float qscale, bf16* Qo, bf16* Ko, bf16* Vto,
                               hipStream_t stream);
int layer_norm_bf16(const bf16* x, int64_t ldx, const float* g, const float* b, bf16* y, int64_t ldy, int rows,
                    int cols, float eps, hipStream_t stream);
int pos_embed_bf16(const bf16* table, const int* idx, const float* wts, bf16* y, int n_tok, int dim,
                   hipStream_t stream);
int row_stats_bf16(const bf16* x, int64_t ldx, int rows, int cols, float eps, f32x2* stats, hipStream_t stream);
int fold_ln_weight_bf16(const bf16* w, int64_t k, int64_t n_pad, const float* gamma, const float* beta, bf16* out,
                        f32x2* cd, hipStream_t stream);
int rotary_table(const int* pos_hw, int n_tok, int head_dim, const float* inv_freq, int round16, f32x2* cs,
                 hipStream_t stream);
int cast_f32_bf16(const float* x, bf16* y, int64_t n, hipStream_t stream);
int gemm_f32(GemmF32Params p, int epi, hipStream_t stream);
int layer_norm_f32(const float* x, int64_t ldx, const float* g, const float* b, float* y, int64_t ldy, int rows,
                   int cols, float eps, hipStream_t stream);
int pos_embed_f32(const float* table, const int* idx, const float* wts, float* y, int n_tok, int dim,
                  hipStream_t stream);
int pack_weight_f32(const float* w, int64_t k_in, int64_t n_out, float* out, hipStream_t stream);
int attention_relayout_f32(const float* q, const float* k, const float* v, int64_t ld, const f32x2* cs, int N, int Np,
                           int H, int hd, int vrows, float qscale, float* Qo, float* Ko, float* Vto,
                           hipStream_t stream);
// fp32 attention on a work list; a split list (items [n_whole, n_items) are key parts) writes the
// parts' partials to `part` (attn_partial_floats(hd) per part) and combines them.
int attention_f32(const float* Qb, const float* Kb, const float* Vtb, const int* d_items, int64_t n_items, int Np,
                  int hd, float* out, int64_t ldo, hipStream_t stream, int64_t n_whole = -1, float* part = nullptr);
int attention_combine_f32(const int* d_tiles, int64_t n_tiles, int64_t n_whole, const float* part, float* out,
                          int64_t ldo, int hd, hipStream_t stream);
int pack_weight_bf16(const float* w, int64_t k_in, int64_t n_out, bf16* out, hipStream_t stream);
// qvl_gather_rows with the identity order when idx is NULL and out columns [width, pad_to) zeroed.
int gather_rows_pad(void* stream, int32_t src_dtype, const void* src, int64_t ld_src, int32_t dst_dtype, void* dst,
                    int64_t ld_dst, const int32_t* idx, int64_t n_rows, int32_t group, int64_t width, int64_t pad_to);

}  // namespace qvl
