// Host side of libqvl that drives the GPU: the C-ABI stage entries (argument checks, launches) and
// the whole-tower orchestration (Qwen3VisionTransformer.__call__). The GPU-free host code (error
// plumbing, integer metadata, work lists) lives in qvl_meta.cpp.
#include <math.h>
#include <string.h>

#include <algorithm>
#include <vector>

#include "qvl_kernels.h"

namespace qvl {

int check_launch(const char* what) {
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) return set_error(QVL_ERR_LAUNCH, "%s: %s", what, hipGetErrorString(e));
  return QVL_OK;
}

static bool aligned16(const void* p) { return ((uintptr_t)p & 15) == 0; }

constexpr float kLog2e = 1.4426950408889634f;

}  // namespace qvl

using namespace qvl;

extern "C" {

// ---------------------------------------------------------------------------------------------
// device stages
// ---------------------------------------------------------------------------------------------
int qvl_pack_dense_weight(void* stream, int32_t dtype, const float* w, int64_t k_in, int64_t n_out, void* out) {
  if (dtype != QVL_DTYPE_BF16 && dtype != QVL_DTYPE_F32) return set_error(QVL_ERR_UNSUPPORTED, "pack: dtype %d", dtype);
  if (!w || !out || k_in <= 0 || n_out <= 0) return set_error(QVL_ERR_INVALID_ARG, "pack: bad args");
  if (dtype == QVL_DTYPE_F32) return pack_weight_f32(w, k_in, n_out, (float*)out, (hipStream_t)stream);
  return pack_weight_bf16(w, k_in, n_out, (bf16*)out, (hipStream_t)stream);
}

int qvl_cast(void* stream, int32_t dtype, const float* x, void* y, int64_t n) {
  if (dtype != QVL_DTYPE_BF16) return set_error(QVL_ERR_UNSUPPORTED, "cast: dtype %d", dtype);
  if (n < 0 || (n > 0 && (!x || !y))) return set_error(QVL_ERR_INVALID_ARG, "cast: bad args");
  if (!aligned16(x) || !aligned16(y)) return set_error(QVL_ERR_MISALIGNED, "cast: pointers must be 16-byte aligned");
  return cast_f32_bf16(x, (bf16*)y, n, (hipStream_t)stream);
}

static int dense_impl(void* stream, int32_t dtype, int32_t epi, const void* x, int64_t lda, const void* w,
                      const float* bias, const void* res, int64_t ldr, void* y, int64_t ldc, int64_t m, int64_t n,
                      int64_t k, void* ws, size_t ws_bytes, const float* ln_cd = nullptr,
                      const float* ln_stats = nullptr, const float* ln_part = nullptr, int ln_groups = 0,
                      float ln_eps = 0.f, float* rs_part = nullptr) {
  if (dtype != QVL_DTYPE_BF16 && dtype != QVL_DTYPE_F32) return set_error(QVL_ERR_UNSUPPORTED, "dense: dtype %d", dtype);
  if (epi < QVL_EPI_BIAS || epi > QVL_EPI_BIAS_RESIDUAL) return set_error(QVL_ERR_INVALID_ARG, "dense: epilogue %d", epi);
  if (m < 0 || n <= 0 || k <= 0) return set_error(QVL_ERR_INVALID_ARG, "dense: m=%lld n=%lld k=%lld", (long long)m, (long long)n, (long long)k);
  if (m == 0) return QVL_OK;
  if (k % 64) return set_error(QVL_ERR_INVALID_ARG, "dense: k=%lld must be a multiple of 64 (pad the weights)", (long long)k);
  if (n % 4) return set_error(QVL_ERR_INVALID_ARG, "dense: n=%lld must be a multiple of 4", (long long)n);
  if (!x || !w || !bias || !y || (epi == QVL_EPI_BIAS_RESIDUAL && !res))
    return set_error(QVL_ERR_INVALID_ARG, "dense: NULL operand");
  if (lda < k || ldc < n || (epi == QVL_EPI_BIAS_RESIDUAL && ldr < n))
    return set_error(QVL_ERR_INVALID_ARG, "dense: leading dimension too small");
  if (dtype == QVL_DTYPE_F32) {
    // fp32: x [m, lda], packed w [round_up(n, 64), k], y / res [m, ld] fp32, 16-byte rows
    if (!aligned16(x) || !aligned16(w) || !aligned16(bias) || !aligned16(y) || lda % 4 || ldc % 4 ||
        (epi == QVL_EPI_BIAS_RESIDUAL && (!aligned16(res) || ldr % 4)) || (ws && !aligned16(ws)))
      return set_error(QVL_ERR_MISALIGNED, "dense: fp32 operands must be 16-byte aligned (lda, ldc, ldr % 4 == 0)");
    if (m * lda * 4 >= (int64_t)UINT32_MAX || round_up(n, 64) * k * 4 >= (int64_t)UINT32_MAX)
      return set_error(QVL_ERR_UNSUPPORTED, "dense: operand larger than 4 GiB");
    GemmF32Params p{};
    p.x = (const float*)x; p.lda = lda; p.w = (const float*)w; p.ldw = k; p.n_rows_w = round_up(n, 64);
    p.bias = bias; p.res = (const float*)res; p.ldr = ldr; p.y = (float*)y; p.ldc = ldc;
    p.M = (int)m; p.N = (int)n; p.K = (int)k; p.Kp = (int)k;
    p.part = (float*)ws; p.part_elems = ws ? (int64_t)(ws_bytes / sizeof(float)) : 0;
    return gemm_f32(p, epi, (hipStream_t)stream);
  }
  if (!aligned16(x) || !aligned16(w) || !aligned16(bias) || !aligned16(y) || lda % 8 || ldc % 4 ||
      (epi == QVL_EPI_BIAS_RESIDUAL && (((uintptr_t)res & 7) || ldr % 4)) || (ws && !aligned16(ws)))
    return set_error(QVL_ERR_MISALIGNED, "dense: operands must be 16-byte aligned (lda % 8 == 0, ldc % 4 == 0)");
  if (m * lda * 2 >= (int64_t)UINT32_MAX || n * k * 2 >= (int64_t)UINT32_MAX)
    return set_error(QVL_ERR_UNSUPPORTED, "dense: operand larger than 4 GiB");
  GemmParams p{};
  p.x = (const bf16*)x; p.lda = lda; p.w = (const bf16*)w; p.bias = bias;
  p.res = (const bf16*)res; p.ldr = ldr; p.y = (bf16*)y; p.ldc = ldc;
  p.M = (int)m; p.N = (int)n; p.K = (int)k;
  p.part = (float*)ws; p.part_elems = ws ? (int64_t)(ws_bytes / sizeof(float)) : 0;
  p.ln_stats = (const f32x2*)ln_stats;
  p.ln_cd = (const f32x2*)ln_cd;
  p.ln_part = (const f32x2*)ln_part;
  p.ln_groups = ln_groups;
  p.ln_eps = ln_eps;
  p.rs_part = (f32x2*)rs_part;
  return gemm_bf16(p, epi, (hipStream_t)stream);
}

int qvl_dense(void* stream, int32_t dtype, int32_t epi, const void* x, int64_t lda, const void* w, const float* bias,
              const void* res, int64_t ldr, void* y, int64_t ldc, int64_t m, int64_t n, int64_t k) {
  return dense_impl(stream, dtype, epi, x, lda, w, bias, res, ldr, y, ldc, m, n, k, nullptr, 0);
}

int qvl_set_gemm_plan(int32_t tile, int32_t split_mode, int32_t group_n) {
  return gemm_set_plan(tile, split_mode, group_n);
}

int qvl_set_attention_plan(int32_t key_groups) { return attention_set_plan(key_groups); }

int qvl_dense_workspace_size(size_t* bytes) {
  if (!bytes) return set_error(QVL_ERR_INVALID_ARG, "bytes is NULL");
  *bytes = (size_t)gemm_partials_elems(gemm_device_cus()) * sizeof(float);
  return QVL_OK;
}

int qvl_dense_ws(void* stream, int32_t dtype, int32_t epi, const void* x, int64_t lda, const void* w, const float* bias,
                 const void* res, int64_t ldr, void* y, int64_t ldc, int64_t m, int64_t n, int64_t k, void* ws,
                 size_t ws_bytes) {
  return dense_impl(stream, dtype, epi, x, lda, w, bias, res, ldr, y, ldc, m, n, k, ws, ws_bytes);
}

int qvl_row_stats(void* stream, int32_t dtype, const void* x, int64_t ldx, int64_t rows, int64_t cols, float eps,
                  float* stats) {
  if (dtype != QVL_DTYPE_BF16) return set_error(QVL_ERR_UNSUPPORTED, "row_stats: dtype %d (bf16 only)", dtype);
  if (rows < 0 || cols <= 0 || cols % 8 || cols > 8192 || ldx < cols || rows > INT32_MAX)
    return set_error(QVL_ERR_INVALID_ARG, "row_stats: rows=%lld cols=%lld", (long long)rows, (long long)cols);
  if (rows == 0) return QVL_OK;
  if (!x || !stats) return set_error(QVL_ERR_INVALID_ARG, "row_stats: NULL operand");
  if (!aligned16(x) || ldx % 8 || ((uintptr_t)stats & 7)) return set_error(QVL_ERR_MISALIGNED, "row_stats: alignment");
  return row_stats_bf16((const bf16*)x, ldx, (int)rows, (int)cols, eps, (f32x2*)stats, (hipStream_t)stream);
}

int qvl_fold_ln_weight(void* stream, int32_t dtype, const void* w, int64_t k_in, int64_t n_out, const float* gamma,
                       const float* beta, void* out_w, float* out_cd) {
  if (dtype != QVL_DTYPE_BF16) return set_error(QVL_ERR_UNSUPPORTED, "fold_ln_weight: dtype %d (bf16 only)", dtype);
  if (k_in <= 0 || k_in % 64 || n_out <= 0 || k_in > INT32_MAX || round_up(n_out, 64) > INT32_MAX)
    return set_error(QVL_ERR_INVALID_ARG, "fold_ln_weight: k_in=%lld (a multiple of 64) n_out=%lld", (long long)k_in,
                     (long long)n_out);
  if (!w || !gamma || !beta || !out_w || !out_cd) return set_error(QVL_ERR_INVALID_ARG, "fold_ln_weight: NULL operand");
  if (!aligned16(w) || !aligned16(gamma) || !aligned16(beta) || !aligned16(out_w) || !aligned16(out_cd))
    return set_error(QVL_ERR_MISALIGNED, "fold_ln_weight: operands must be 16-byte aligned");
  return fold_ln_weight_bf16((const bf16*)w, k_in, round_up(n_out, 64), gamma, beta, (bf16*)out_w, (f32x2*)out_cd,
                             (hipStream_t)stream);
}

int qvl_dense_ln_ws(void* stream, int32_t dtype, int32_t epi, const void* x, int64_t lda, const void* w,
                    const float* cd, const float* stats, const float* bias, void* y, int64_t ldc, int64_t m, int64_t n,
                    int64_t k, void* ws, size_t ws_bytes) {
  if (dtype != QVL_DTYPE_BF16) return set_error(QVL_ERR_UNSUPPORTED, "dense_ln: dtype %d (bf16 only)", dtype);
  if (epi != QVL_EPI_BIAS && epi != QVL_EPI_BIAS_GELU)
    return set_error(QVL_ERR_INVALID_ARG, "dense_ln: epilogue %d (bias or bias+GELU)", epi);
  if (m > 0 && (!cd || !stats)) return set_error(QVL_ERR_INVALID_ARG, "dense_ln: NULL folded LayerNorm operand");
  if (((uintptr_t)cd & 15) || ((uintptr_t)stats & 7)) return set_error(QVL_ERR_MISALIGNED, "dense_ln: alignment");
  return dense_impl(stream, dtype, epi, x, lda, w, bias, nullptr, 0, y, ldc, m, n, k, ws, ws_bytes, cd, stats);
}

int qvl_layer_norm(void* stream, int32_t dtype, const void* x, int64_t ldx, const float* g, const float* b, void* y,
                   int64_t ldy, int64_t rows, int64_t cols, float eps) {
  if (dtype != QVL_DTYPE_BF16 && dtype != QVL_DTYPE_F32) return set_error(QVL_ERR_UNSUPPORTED, "layer_norm: dtype %d", dtype);
  if (rows < 0 || cols <= 0 || cols % 8 || cols > 8192 || ldx < cols || ldy < cols)
    return set_error(QVL_ERR_INVALID_ARG, "layer_norm: rows=%lld cols=%lld", (long long)rows, (long long)cols);
  if (!x || !g || !b || !y) return set_error(QVL_ERR_INVALID_ARG, "layer_norm: NULL operand");
  if (dtype == QVL_DTYPE_F32) {
    if (!aligned16(x) || !aligned16(y) || !aligned16(g) || !aligned16(b) || ldx % 4 || ldy % 4)
      return set_error(QVL_ERR_MISALIGNED, "layer_norm: operands must be 16-byte aligned");
    return layer_norm_f32((const float*)x, ldx, g, b, (float*)y, ldy, (int)rows, (int)cols, eps, (hipStream_t)stream);
  }
  if (!aligned16(x) || !aligned16(y) || !aligned16(g) || !aligned16(b) || ldx % 8 || ldy % 8)
    return set_error(QVL_ERR_MISALIGNED, "layer_norm: operands must be 16-byte aligned");
  return layer_norm_bf16((const bf16*)x, ldx, g, b, (bf16*)y, ldy, (int)rows, (int)cols, eps, (hipStream_t)stream);
}

int qvl_pos_embed(void* stream, int32_t dtype, const void* table, const int32_t* idx, const float* w, void* y,
                  int64_t n_tokens, int64_t dim) {
  if (dtype != QVL_DTYPE_BF16 && dtype != QVL_DTYPE_F32) return set_error(QVL_ERR_UNSUPPORTED, "pos_embed: dtype %d", dtype);
  if (n_tokens < 0 || dim <= 0 || dim % 8) return set_error(QVL_ERR_INVALID_ARG, "pos_embed: dim=%lld", (long long)dim);
  if (!table || !idx || !w || !y) return set_error(QVL_ERR_INVALID_ARG, "pos_embed: NULL operand");
  if (!aligned16(table) || !aligned16(y)) return set_error(QVL_ERR_MISALIGNED, "pos_embed: operands must be 16-byte aligned");
  if (dtype == QVL_DTYPE_F32)
    return pos_embed_f32((const float*)table, idx, w, (float*)y, (int)n_tokens, (int)dim, (hipStream_t)stream);
  return pos_embed_bf16((const bf16*)table, idx, w, (bf16*)y, (int)n_tokens, (int)dim, (hipStream_t)stream);
}

int qvl_rotary_table(void* stream, int32_t dtype, const int32_t* pos_hw, int64_t n_tokens, int32_t head_dim, float theta,
                     void* cs) {
  if (dtype != QVL_DTYPE_BF16 && dtype != QVL_DTYPE_F32) return set_error(QVL_ERR_INVALID_ARG, "rotary: dtype %d", dtype);
  float inv[32];
  int rc = qvl_rotary_inv_freq(head_dim, theta, inv);
  if (rc) return rc;
  if (n_tokens < 0 || (n_tokens > 0 && (!pos_hw || !cs))) return set_error(QVL_ERR_INVALID_ARG, "rotary: bad args");
  return rotary_table(pos_hw, (int)n_tokens, head_dim, inv, dtype == QVL_DTYPE_BF16, (f32x2*)cs, (hipStream_t)stream);
}

static int64_t attn_np(int64_t n) { return round_up(std::max<int64_t>(n, 1), 64); }

// Head-major attention operand geometry: Q/K rows of `hdp` dims, V^T of `vrows` rows. bf16
// head_dim 72 stores Q/K rows of 88 (176 bytes, the hd-72 kernel's DMA / LDS row) and V^T rows
// 0..71; fp32 keeps Q/K exact and pads V^T to 32-row blocks.
static int attn_dims(int dtype, int hd, int* hdp, int* vrows) {
  if (hd != 64 && hd != 72 && hd != 80)
    return set_error(QVL_ERR_UNSUPPORTED, "attention: head_dim=%d (supported: 64, 72, 80)", hd);
  if (dtype == QVL_DTYPE_F32) { *hdp = hd; *vrows = (int)round_up(hd, 32); return QVL_OK; }
  if (dtype != QVL_DTYPE_BF16) return set_error(QVL_ERR_UNSUPPORTED, "attention: dtype %d", dtype);
  *hdp = hd == 64 ? 64 : 88;
  *vrows = hd;
  return QVL_OK;
}

static size_t dtype_size(int dtype) { return dtype == QVL_DTYPE_F32 ? 4 : 2; }

int qvl_vision_attention_workspace_size(int32_t dtype, int64_t n_tokens, int32_t num_heads, int32_t head_dim,
                                        size_t* bytes) {
  if (!bytes || n_tokens < 0 || num_heads <= 0) return set_error(QVL_ERR_INVALID_ARG, "attention ws: bad args");
  int hdp, vrows;
  int rc = attn_dims(dtype, head_dim, &hdp, &vrows);
  if (rc) return rc;
  *bytes = (size_t)num_heads * attn_np(n_tokens) * (2 * hdp + vrows) * dtype_size(dtype);
  return QVL_OK;
}

int qvl_vision_attention(void* stream, int32_t dtype, const void* q, const void* k, const void* v, int64_t ld,
                         const void* cs, const int32_t* tiles, int64_t n_tiles, void* out, int64_t ld_out,
                         int64_t n_tokens, int32_t H, int32_t hd, void* ws, size_t ws_bytes) {
  size_t need = 0;
  int rc = qvl_vision_attention_workspace_size(dtype, n_tokens, H, hd, &need);
  if (rc) return rc;
  if (ws_bytes < need || !ws) return set_error(QVL_ERR_WORKSPACE, "attention: workspace %zu < %zu", ws_bytes, need);
  if (n_tokens == 0) return QVL_OK;
  if (!q || !k || !v || !cs || !out || (n_tiles > 0 && !tiles)) return set_error(QVL_ERR_INVALID_ARG, "attention: NULL operand");
  if (ld < (int64_t)H * hd || ld_out < (int64_t)H * hd || ld_out % 4)
    return set_error(QVL_ERR_INVALID_ARG, "attention: leading dimensions");
  if (((uintptr_t)out & 7) || !aligned16(ws)) return set_error(QVL_ERR_MISALIGNED, "attention: alignment");
  const int64_t Np = attn_np(n_tokens);
  int hdp, vrows;
  attn_dims(dtype, hd, &hdp, &vrows);
  if (dtype == QVL_DTYPE_F32) {
    if (!aligned16(q) || !aligned16(k) || !aligned16(v) || ld % 4 || !aligned16(out))
      return set_error(QVL_ERR_MISALIGNED, "attention: fp32 operands must be 16-byte aligned");
    float* Qf = (float*)ws;
    float* Kf = Qf + (size_t)H * Np * hdp;
    float* Vf = Kf + (size_t)H * Np * hdp;
    rc = attention_relayout_f32((const float*)q, (const float*)k, (const float*)v, ld, (const f32x2*)cs, (int)n_tokens,
                                (int)Np, H, hd, vrows, (1.0f / sqrtf((float)hd)) * kLog2e, Qf, Kf, Vf, (hipStream_t)stream);
    if (rc) return rc;
    return attention_f32(Qf, Kf, Vf, tiles, n_tiles, (int)Np, hd, (float*)out, ld_out, (hipStream_t)stream);
  }
  bf16* Qb = (bf16*)ws;
  bf16* Kb = Qb + (size_t)H * Np * hdp;
  bf16* Vb = Kb + (size_t)H * Np * hdp;
  const float qscale = (1.0f / sqrtf((float)hd)) * kLog2e;
  if (hd == 64) {
    rc = attention_relayout_hd64((const bf16*)q, (const bf16*)k, (const bf16*)v, ld, (const f32x2*)cs, (int)n_tokens,
                                 (int)Np, H, qscale, Qb, Kb, Vb, (hipStream_t)stream);
    if (rc) return rc;
    return attention_hd64(Qb, Kb, Vb, tiles, n_tiles, (int)Np, H, (bf16*)out, ld_out, (hipStream_t)stream);
  }
  rc = attention_relayout_general((const bf16*)q, (const bf16*)k, (const bf16*)v, ld, (const f32x2*)cs, (int)n_tokens,
                                  (int)Np, H, hd, hdp, vrows, qscale, Qb, Kb, Vb, (hipStream_t)stream);
  if (rc) return rc;
  return attention_general(Qb, Kb, Vb, tiles, n_tiles, (int)Np, H, hd, (bf16*)out, ld_out, (hipStream_t)stream);
}

int qvl_rotary_pos_table(void* stream, int32_t head_dim, float theta, int32_t n_positions, uint32_t* table) {
  float inv[32];
  QVL_TRY_RC(qvl_rotary_inv_freq(head_dim, theta, inv));
  if (n_positions < 0 || (n_positions > 0 && !table)) return set_error(QVL_ERR_INVALID_ARG, "rotary_pos_table: bad args");
  return rotary_pos_table(n_positions, head_dim, inv, table, (hipStream_t)stream);
}

static int qkv_rotary_impl(void* stream, int32_t dtype, const void* x, int64_t lda, const void* w, const float* bias,
                           const void* cs, const int32_t* pos_hw, const uint32_t* rtab, int32_t n_pos, void* q,
                           void* k, void* vt, int64_t n_tokens, int64_t hidden, int32_t H, void* ws, size_t ws_bytes,
                           const float* ln_cd = nullptr, const float* ln_stats = nullptr,
                           const float* ln_part = nullptr, int ln_groups = 0, float ln_eps = 0.f) {
  if (dtype != QVL_DTYPE_BF16) return set_error(QVL_ERR_UNSUPPORTED, "qkv_rotary: dtype %d", dtype);
  const bool ln = ln_stats || ln_part;
  if (H <= 0 || (hidden != (int64_t)H * 64 && hidden != (int64_t)H * 72))
    return set_error(QVL_ERR_UNSUPPORTED, "qkv_rotary: head_dim must be 64 or 72");
  const int hd = (int)(hidden / H);
  if (hd == 64 && hidden % 128) return set_error(QVL_ERR_UNSUPPORTED, "qkv_rotary: hidden %% 128 != 0");
  if (hd == 72 && H % 4) return set_error(QVL_ERR_UNSUPPORTED, "qkv_rotary: head_dim 72 needs num_heads %% 4 == 0");
  if (n_tokens < 0 || lda < hidden || lda % 8) return set_error(QVL_ERR_INVALID_ARG, "qkv_rotary: n_tokens / lda");
  if (n_tokens == 0) return QVL_OK;
  if (!x || !w || !bias || !q || !k || !vt || (!cs && (!pos_hw || !rtab)))
    return set_error(QVL_ERR_INVALID_ARG, "qkv_rotary: NULL operand");
  if (rtab && (n_pos <= 0 || (int64_t)n_pos * (hd / 4) * 4 > rope_table_lds_bytes(hd, ln)))
    return set_error(QVL_ERR_UNSUPPORTED, "qkv_rotary: %d rotary positions exceed the %d-byte table of head_dim %d",
                     n_pos, rope_table_lds_bytes(hd, ln), hd);
  if (!aligned16(x) || !aligned16(w) || !aligned16(bias) || !aligned16(q) || !aligned16(k) || !aligned16(vt) ||
      (cs && !aligned16(cs)) || (rtab && !aligned16(rtab)))
    return set_error(QVL_ERR_MISALIGNED, "qkv_rotary: alignment");
  if (n_tokens * lda * 2 >= (int64_t)UINT32_MAX) return set_error(QVL_ERR_UNSUPPORTED, "qkv_rotary: operand > 4 GiB");
  GemmParams p{};
  p.x = (const bf16*)x; p.lda = lda; p.w = (const bf16*)w; p.bias = bias;
  p.M = (int)n_tokens; p.N = (int)(3 * hidden); p.K = (int)hidden;
  p.q = (bf16*)q; p.k = (bf16*)k; p.vt = (bf16*)vt;
  p.cs = rtab ? nullptr : (const f32x2*)cs;
  p.pos_hw = rtab ? pos_hw : nullptr;
  p.rtab = rtab;
  p.rtab_pos = rtab ? n_pos : 0;
  p.Np = (int)attn_np(n_tokens); p.D = (int)hidden;
  p.cs_half = hd / 2;
  p.qscale = (1.0f / sqrtf((float)hd)) * kLog2e;
  if (ws && !aligned16(ws)) return set_error(QVL_ERR_MISALIGNED, "qkv_rotary: workspace alignment");
  p.part = (float*)ws; p.part_elems = ws ? (int64_t)(ws_bytes / sizeof(float)) : 0;
  p.ln_stats = (const f32x2*)ln_stats;
  p.ln_cd = (const f32x2*)ln_cd;
  p.ln_part = (const f32x2*)ln_part;
  p.ln_groups = ln_groups;
  p.ln_eps = ln_eps;
  return gemm_bf16(p, hd == 64 ? kEpiQkvRope : kEpiQkvRope72, (hipStream_t)stream);
}

int qvl_dense_qkv_rotary(void* stream, int32_t dtype, const void* x, int64_t lda, const void* w, const float* bias,
                         const void* cs, void* q, void* k, void* vt, int64_t n_tokens, int64_t hidden, int32_t H,
                         void* ws, size_t ws_bytes) {
  if (n_tokens > 0 && !cs) return set_error(QVL_ERR_INVALID_ARG, "qkv_rotary: NULL cos/sin table");
  return qkv_rotary_impl(stream, dtype, x, lda, w, bias, cs, nullptr, nullptr, 0, q, k, vt, n_tokens, hidden, H, ws,
                         ws_bytes);
}

int qvl_dense_qkv_rotary_pos(void* stream, int32_t dtype, const void* x, int64_t lda, const void* w, const float* bias,
                             const int32_t* pos_hw, const uint32_t* table, int32_t n_positions, void* q, void* k,
                             void* vt, int64_t n_tokens, int64_t hidden, int32_t H, void* ws, size_t ws_bytes) {
  if (n_tokens > 0 && (!pos_hw || !table)) return set_error(QVL_ERR_INVALID_ARG, "qkv_rotary_pos: NULL positions/table");
  return qkv_rotary_impl(stream, dtype, x, lda, w, bias, nullptr, pos_hw, table, n_positions, q, k, vt, n_tokens,
                         hidden, H, ws, ws_bytes);
}

int qvl_dense_qkv_rotary_ln(void* stream, int32_t dtype, const void* x, int64_t lda, const void* w, const float* cd,
                            const float* stats, const float* bias, const void* cs, const int32_t* pos_hw,
                            const uint32_t* table, int32_t n_positions, void* q, void* k, void* vt, int64_t n_tokens,
                            int64_t hidden, int32_t H, void* ws, size_t ws_bytes) {
  if (n_tokens > 0 && (!cd || !stats)) return set_error(QVL_ERR_INVALID_ARG, "qkv_rotary_ln: NULL folded LayerNorm operand");
  if (((uintptr_t)cd & 15) || ((uintptr_t)stats & 7)) return set_error(QVL_ERR_MISALIGNED, "qkv_rotary_ln: alignment");
  if (n_tokens > 0 && (cs ? (pos_hw || table) : (!pos_hw || !table)))
    return set_error(QVL_ERR_INVALID_ARG, "qkv_rotary_ln: give either the per-token cos/sin table or positions + table");
  return qkv_rotary_impl(stream, dtype, x, lda, w, bias, cs, cs ? nullptr : pos_hw, cs ? nullptr : table,
                         cs ? 0 : n_positions, q, k, vt, n_tokens, hidden, H, ws, ws_bytes, cd, stats);
}

// Row-statistics partials of a LayerNorm's input (128-column groups): shared argument checks.
static int check_ln_parts(const char* what, int64_t rows, int64_t cols, const float* cd, const float* parts,
                          int32_t groups, float eps) {
  if (rows > 0 && (!cd || !parts)) return set_error(QVL_ERR_INVALID_ARG, "%s: NULL folded LayerNorm operand", what);
  if (groups <= 0 || groups > 64 || (int64_t)groups * 128 != cols)
    return set_error(QVL_ERR_INVALID_ARG, "%s: %d 128-column groups for rows of %lld", what, groups, (long long)cols);
  if (!(eps > 0.f)) return set_error(QVL_ERR_INVALID_ARG, "%s: eps must be positive", what);
  if (((uintptr_t)cd & 15) || ((uintptr_t)parts & 7)) return set_error(QVL_ERR_MISALIGNED, "%s: alignment", what);
  return QVL_OK;
}

int qvl_dense_rowstats_ws(void* stream, int32_t dtype, const void* x, int64_t lda, const void* w, const float* bias,
                          const void* res, int64_t ldr, void* y, int64_t ldc, int64_t m, int64_t n, int64_t k,
                          float* parts, void* ws, size_t ws_bytes) {
  if (dtype != QVL_DTYPE_BF16) return set_error(QVL_ERR_UNSUPPORTED, "dense_rowstats: dtype %d (bf16 only)", dtype);
  if (n % 128) return set_error(QVL_ERR_UNSUPPORTED, "dense_rowstats: n=%lld not a multiple of 128", (long long)n);
  if (m > 0 && !parts) return set_error(QVL_ERR_INVALID_ARG, "dense_rowstats: NULL partials");
  if (((uintptr_t)parts & 7) || ldc % 8 || ldr % 8)
    return set_error(QVL_ERR_MISALIGNED, "dense_rowstats: partials 8-byte aligned, ldc and ldr multiples of 8");
  return dense_impl(stream, dtype, QVL_EPI_BIAS_RESIDUAL, x, lda, w, bias, res, ldr, y, ldc, m, n, k, ws, ws_bytes,
                    nullptr, nullptr, nullptr, 0, 0.f, parts);
}

int qvl_dense_pos_embed_ws(void* stream, int32_t dtype, const void* x, int64_t lda, const void* w, const float* bias,
                           const void* table, const int32_t* tap_idx, const float* tap_w, void* y, int64_t ldc,
                           int64_t m, int64_t n, int64_t k, float* parts, void* ws, size_t ws_bytes) {
  (void)ws;
  (void)ws_bytes;
  if (dtype != QVL_DTYPE_BF16) return set_error(QVL_ERR_UNSUPPORTED, "dense_pos_embed: dtype %d (bf16 only)", dtype);
  if (m < 0 || n <= 0 || k <= 0 || k % 64 || n % 8)
    return set_error(QVL_ERR_INVALID_ARG, "dense_pos_embed: m=%lld n=%lld (multiple of 8) k=%lld (multiple of 64)",
                     (long long)m, (long long)n, (long long)k);
  if (m == 0) return QVL_OK;
  if (!x || !w || !bias || !y || !table || !tap_idx || !tap_w)
    return set_error(QVL_ERR_INVALID_ARG, "dense_pos_embed: NULL operand");
  if (lda < k || ldc < n) return set_error(QVL_ERR_INVALID_ARG, "dense_pos_embed: leading dimension too small");
  if (parts && n % 128)
    return set_error(QVL_ERR_UNSUPPORTED, "dense_pos_embed: row partials need n %% 128 == 0 (n=%lld)", (long long)n);
  if (!aligned16(x) || !aligned16(w) || !aligned16(bias) || !aligned16(y) || !aligned16(table) || lda % 8 ||
      ldc % 8 || ((uintptr_t)parts & 7) || ((uintptr_t)tap_idx & 3) || ((uintptr_t)tap_w & 3))
    return set_error(QVL_ERR_MISALIGNED, "dense_pos_embed: operands 16-byte aligned, lda and ldc multiples of 8");
  if (m * lda * 2 >= (int64_t)UINT32_MAX || n * k * 2 >= (int64_t)UINT32_MAX)
    return set_error(QVL_ERR_UNSUPPORTED, "dense_pos_embed: operand larger than 4 GiB");
  GemmParams p{};
  p.x = (const bf16*)x; p.lda = lda; p.w = (const bf16*)w; p.bias = bias;
  p.y = (bf16*)y; p.ldc = ldc;
  p.M = (int)m; p.N = (int)n; p.K = (int)k;
  p.rs_part = (f32x2*)parts;
  p.pe_table = (const bf16*)table;
  p.pe_idx = tap_idx;
  p.pe_w = tap_w;
  return gemm_bf16(p, kEpiBiasPosEmbed, (hipStream_t)stream);
}

int qvl_dense_ln_parts_ws(void* stream, int32_t dtype, int32_t epi, const void* x, int64_t lda, const void* w,
                          const float* cd, const float* parts, int32_t groups, float eps, const float* bias, void* y,
                          int64_t ldc, int64_t m, int64_t n, int64_t k, void* ws, size_t ws_bytes) {
  if (dtype != QVL_DTYPE_BF16) return set_error(QVL_ERR_UNSUPPORTED, "dense_ln_parts: dtype %d (bf16 only)", dtype);
  if (epi != QVL_EPI_BIAS && epi != QVL_EPI_BIAS_GELU)
    return set_error(QVL_ERR_INVALID_ARG, "dense_ln_parts: epilogue %d (bias or bias+GELU)", epi);
  QVL_TRY_RC(check_ln_parts("dense_ln_parts", m, k, cd, parts, groups, eps));
  return dense_impl(stream, dtype, epi, x, lda, w, bias, nullptr, 0, y, ldc, m, n, k, ws, ws_bytes, cd, nullptr,
                    parts, groups, eps);
}

int qvl_dense_qkv_rotary_ln_parts(void* stream, int32_t dtype, const void* x, int64_t lda, const void* w,
                                  const float* cd, const float* parts, int32_t groups, float eps, const float* bias,
                                  const void* cs, const int32_t* pos_hw, const uint32_t* table, int32_t n_positions,
                                  void* q, void* k, void* vt, int64_t n_tokens, int64_t hidden, int32_t H, void* ws,
                                  size_t ws_bytes) {
  QVL_TRY_RC(check_ln_parts("qkv_rotary_ln_parts", n_tokens, hidden, cd, parts, groups, eps));
  if (n_tokens > 0 && (cs ? (pos_hw || table) : (!pos_hw || !table)))
    return set_error(QVL_ERR_INVALID_ARG, "qkv_rotary_ln_parts: give either the per-token cos/sin table or positions + table");
  return qkv_rotary_impl(stream, dtype, x, lda, w, bias, cs, cs ? nullptr : pos_hw, cs ? nullptr : table,
                         cs ? 0 : n_positions, q, k, vt, n_tokens, hidden, H, ws, ws_bytes, cd, nullptr, parts, groups,
                         eps);
}

int qvl_attention_headmajor(void* stream, int32_t dtype, const void* q, const void* k, const void* vt,
                            const int32_t* tiles, int64_t n_tiles, int64_t n_tokens, int32_t H, int32_t hd, void* out,
                            int64_t ld_out) {
  int hdp, vrows;
  int rc = attn_dims(dtype, hd, &hdp, &vrows);
  if (rc) return rc;
  if (n_tokens < 0 || H <= 0 || n_tiles < 0 || ld_out < (int64_t)H * hd || ld_out % 4)
    return set_error(QVL_ERR_INVALID_ARG, "attention: bad sizes");
  if (n_tokens == 0 || n_tiles == 0) return QVL_OK;
  if (!q || !k || !vt || !tiles || !out) return set_error(QVL_ERR_INVALID_ARG, "attention: NULL operand");
  if ((uintptr_t)out & 7) return set_error(QVL_ERR_MISALIGNED, "attention: out alignment");
  if (dtype == QVL_DTYPE_F32) {
    if (!aligned16(out) || ld_out % 4) return set_error(QVL_ERR_MISALIGNED, "attention: fp32 out alignment");
    return attention_f32((const float*)q, (const float*)k, (const float*)vt, tiles, n_tiles, (int)attn_np(n_tokens), hd,
                         (float*)out, ld_out, (hipStream_t)stream);
  }
  if (hd == 64)
    return attention_hd64((const bf16*)q, (const bf16*)k, (const bf16*)vt, tiles, n_tiles, (int)attn_np(n_tokens), H,
                          (bf16*)out, ld_out, (hipStream_t)stream);
  return attention_general((const bf16*)q, (const bf16*)k, (const bf16*)vt, tiles, n_tiles, (int)attn_np(n_tokens), H,
                           hd, (bf16*)out, ld_out, (hipStream_t)stream);
}

int qvl_attention_split_workspace_size(int32_t head_dim, int64_t n_tiles, int64_t n_whole, size_t* bytes) {
  if (!bytes || n_tiles < 0 || n_whole < 0 || n_whole > n_tiles)
    return set_error(QVL_ERR_INVALID_ARG, "attention split ws: bad args");
  if (head_dim != 64 && head_dim != 72 && head_dim != 80)
    return set_error(QVL_ERR_UNSUPPORTED, "attention split: head_dim=%d", head_dim);
  *bytes = (size_t)(n_tiles - n_whole) * attn_partial_floats(head_dim) * sizeof(float);
  return QVL_OK;
}

int qvl_attention_headmajor_split(void* stream, int32_t dtype, const void* q, const void* k, const void* vt,
                                  const int32_t* tiles, int64_t n_tiles, int64_t n_whole, int64_t n_tokens, int32_t H,
                                  int32_t hd, void* out, int64_t ld_out, void* ws, size_t ws_bytes) {
  if (dtype != QVL_DTYPE_BF16 && dtype != QVL_DTYPE_F32)
    return set_error(QVL_ERR_UNSUPPORTED, "attention split: dtype %d", dtype);
  if (hd != 64 && hd != 72 && hd != 80) return set_error(QVL_ERR_UNSUPPORTED, "attention split: head_dim=%d", hd);
  if (n_tokens < 0 || H <= 0 || n_tiles < 0 || n_whole < 0 || n_whole > n_tiles || ld_out < (int64_t)H * hd ||
      ld_out % 4)
    return set_error(QVL_ERR_INVALID_ARG, "attention split: bad sizes");
  if (n_tokens == 0 || n_tiles == 0) return QVL_OK;
  if (!q || !k || !vt || !tiles || !out) return set_error(QVL_ERR_INVALID_ARG, "attention split: NULL operand");
  if ((uintptr_t)out & (dtype == QVL_DTYPE_F32 ? 15 : 7)) return set_error(QVL_ERR_MISALIGNED, "attention split: out alignment");
  const size_t need = (size_t)(n_tiles - n_whole) * attn_partial_floats(hd) * sizeof(float);
  if (need && (!ws || ws_bytes < need)) return set_error(QVL_ERR_WORKSPACE, "attention split: workspace %zu < %zu", ws_bytes, need);
  if (need && !aligned16(ws)) return set_error(QVL_ERR_MISALIGNED, "attention split: workspace alignment");
  const int Np = (int)attn_np(n_tokens);
  if (dtype == QVL_DTYPE_F32) {
    // fp32 operands in qvl_attention_headmajor's fp32 layout
    if (!aligned16(q) || !aligned16(k) || !aligned16(vt)) return set_error(QVL_ERR_MISALIGNED, "attention split: fp32 operands");
    return attention_f32((const float*)q, (const float*)k, (const float*)vt, tiles, n_tiles, Np, hd, (float*)out, ld_out,
                         (hipStream_t)stream, n_whole, need ? (float*)ws : nullptr);
  }
  if (hd == 64)
    return attention_hd64((const bf16*)q, (const bf16*)k, (const bf16*)vt, tiles, n_tiles, Np, H, (bf16*)out, ld_out,
                          (hipStream_t)stream, n_whole, need ? (float*)ws : nullptr);
  return attention_general((const bf16*)q, (const bf16*)k, (const bf16*)vt, tiles, n_tiles, Np, H, hd, (bf16*)out,
                           ld_out, (hipStream_t)stream, n_whole, need ? (float*)ws : nullptr);
}

// ---------------------------------------------------------------------------------------------
// whole tower
// ---------------------------------------------------------------------------------------------
struct TowerLayout {
  int dtype;
  size_t esz;
  int64_t N, Np, D, I_pad, PV, PVp, hd, H;   // PVp: the pixel rows' width in the patch-embed GEMM
  int hdp, vrows;
  size_t off_x, off_xn, off_q, off_k, off_vt, off_h, off_cs, off_part, part_bytes, off_apart, off_stats, apart_bytes, total;
  int stat_groups;   // 128-column groups of a row's LayerNorm partials (hidden / 128; 0: hidden % 128 != 0)
};

// Upper bound on the parts of split attention items one work list holds (qvl_attention_
// worklist_split: at most one per workgroup slot, 4 per CU).
static int64_t attn_split_slots_bound() { return 4 * (int64_t)gemm_device_cus(); }

// Whether the tower's qkv Dense runs qvl_dense_qkv_rotary (rotary + head-major operands in its
// epilogue): bf16 with head_dim 64, or head_dim 72 with whole 4-head tiles.
static bool fused_qkv_rotary(int dtype, int hd, int H) {
  return dtype == QVL_DTYPE_BF16 && (hd == 64 || (hd == 72 && H % 4 == 0));
}

static int tower_layout(const qvl_vision_config* c, int64_t N, TowerLayout* L) {
  if (!c) return set_error(QVL_ERR_INVALID_ARG, "config is NULL");
  if (c->dtype != QVL_DTYPE_BF16 && c->dtype != QVL_DTYPE_F32)
    return set_error(QVL_ERR_UNSUPPORTED, "encode_vision: dtype %d", c->dtype);
  if (c->spatial_merge_size != 2) return set_error(QVL_ERR_UNSUPPORTED, "spatial_merge_size=%d", c->spatial_merge_size);
  if (c->num_heads <= 0 || c->hidden_size % c->num_heads) return set_error(QVL_ERR_INVALID_ARG, "hidden/heads");
  const int64_t hd = c->hidden_size / c->num_heads;
  int hdp, vrows;
  QVL_TRY_RC(attn_dims(c->dtype, (int)hd, &hdp, &vrows));
  if (c->hidden_size % 64 || c->out_hidden_size % 64)
    return set_error(QVL_ERR_UNSUPPORTED, "encode_vision: hidden and out_hidden_size must be multiples of 64");
  if (c->patch_volume <= 0 || c->patch_volume % 4)
    return set_error(QVL_ERR_UNSUPPORTED, "encode_vision: patch_volume=%d (a multiple of 4)", c->patch_volume);
  if (c->dtype == QVL_DTYPE_BF16 && hd == 64 && c->hidden_size % 128)
    return set_error(QVL_ERR_UNSUPPORTED, "encode_vision: hidden %% 128 != 0 with head_dim 64");
  if (c->n_deepstack < 0 || c->n_deepstack > 8) return set_error(QVL_ERR_INVALID_ARG, "n_deepstack=%d", c->n_deepstack);
  if (N % 4) return set_error(QVL_ERR_INVALID_ARG, "n_tokens=%lld not a multiple of 4", (long long)N);
  L->dtype = c->dtype;
  L->esz = dtype_size(c->dtype);
  L->N = N; L->Np = attn_np(N); L->D = c->hidden_size; L->I_pad = round_up(c->intermediate_size, 64);
  L->PV = c->patch_volume; L->hd = hd; L->H = c->num_heads; L->hdp = hdp; L->vrows = vrows;
  // the patch-embed GEMM runs K = the packed patch weight's zero-padded width (a multiple of 64):
  // pixel rows of another width are staged zero-padded to it
  L->PVp = round_up(L->PV, 64);
  const bool fused_qkv = fused_qkv_rotary(c->dtype, (int)hd, c->num_heads);
  // h hosts the bf16 pixels, the MLP hidden, the merger hidden and (unless the qkv GEMM writes
  // head-major operands itself) the qkv output.
  int64_t hcols = std::max<int64_t>({L->I_pad, L->PVp, (int64_t)c->hidden_size});
  if (!fused_qkv) hcols = std::max<int64_t>(hcols, 3 * (int64_t)c->hidden_size);
  const size_t e = L->esz;
  size_t o = 0;
  auto take = [&](size_t bytes) { size_t r = o; o += round_up((int64_t)bytes, 256); return r; };
  L->off_x = take((size_t)N * L->D * e);
  L->off_xn = take((size_t)N * L->D * e);
  L->off_q = take((size_t)L->H * L->Np * hdp * e);
  L->off_k = take((size_t)L->H * L->Np * hdp * e);
  L->off_vt = take((size_t)L->H * L->Np * vrows * e);
  L->off_h = take((size_t)N * hcols * e);
  L->off_cs = take((size_t)N * (hd / 2) * 8);
  L->part_bytes = (size_t)gemm_partials_elems(gemm_device_cus()) * sizeof(float);   // split-K partials (both dtypes)
  L->off_part = take(L->part_bytes);
  // partial outputs of split attention items: at most one per workgroup slot (4 per CU)
  L->apart_bytes = (size_t)attn_split_slots_bound() * attn_partial_floats((int)hd) * 4;   // split attention partials
  L->off_apart = take(L->apart_bytes);
  // row statistics of the LayerNorms folded into the following Dense (bf16): per-128-column partials
  // (sum, squared deviations) of each row of x, or (mean, rstd) per row when hidden % 128 != 0
  L->stat_groups = c->hidden_size % 128 == 0 ? (int)(c->hidden_size / 128) : 0;
  L->off_stats = c->dtype == QVL_DTYPE_BF16 ? take((size_t)N * 8 * std::max(1, L->stat_groups)) : 0;
  L->total = o;
  return QVL_OK;
}

int qvl_encode_vision_workspace_size(const qvl_vision_config* cfg, int64_t n_tokens, size_t* bytes) {
  TowerLayout L;
  int rc = tower_layout(cfg, n_tokens, &L);
  if (rc) return rc;
  if (!bytes) return set_error(QVL_ERR_INVALID_ARG, "bytes is NULL");
  *bytes = L.total;
  return QVL_OK;
}


// VisionPatchMerger.__call__ (model.py:648-656): main (LN over D then view [N/4, 4D]) or
// deepstack (view [N/4, 4D] then LN over 4D); fc1 + GELU-tanh; fc2.
// A deepstack merger in bf16 with its norm folded into fc1 reads the row statistics of x instead of
// running the LayerNorm: the fc2 epilogue's partials of the merged rows' 4 tokens (parts_groups =
// 128-column groups per token row, 0: none), or a qvl_row_stats launch.
static int run_merger(hipStream_t st, const qvl_vision_config* c, const TowerLayout& L, const qvl_merger_weights& mw,
                      bool postshuffle, const void* x, void* xn, void* h, void* out, void* part, float* stats,
                      int parts_groups) {
  const int64_t N = L.N, D = L.D, D4 = 4 * L.D;
  const int dt = L.dtype;
  if (postshuffle && dt == QVL_DTYPE_BF16 && mw.fc1_ln.w && mw.fc1_ln.cd && stats) {
    if (parts_groups > 0 && 4 * parts_groups <= 64) {   // (hidden <= 2048: the merger LayerNorm's width bound)
      QVL_TRY_RC(qvl_dense_ln_parts_ws(st, dt, QVL_EPI_BIAS_GELU, x, D4, mw.fc1_ln.w, mw.fc1_ln.cd, stats,
                                       4 * parts_groups, c->ln_eps, mw.fc1_b, h, D4, N / 4, D4, D4, part, L.part_bytes));
    } else {
      QVL_TRY_RC(qvl_row_stats(st, dt, x, D4, N / 4, D4, c->ln_eps, stats));
      QVL_TRY_RC(qvl_dense_ln_ws(st, dt, QVL_EPI_BIAS_GELU, x, D4, mw.fc1_ln.w, mw.fc1_ln.cd, stats, mw.fc1_b, h, D4,
                                 N / 4, D4, D4, part, L.part_bytes));
    }
  } else {
    if (postshuffle)
      QVL_TRY_RC(qvl_layer_norm(st, dt, x, D4, mw.norm_w, mw.norm_b, xn, D4, N / 4, D4, c->ln_eps));
    else
      QVL_TRY_RC(qvl_layer_norm(st, dt, x, D, mw.norm_w, mw.norm_b, xn, D, N, D, c->ln_eps));
    QVL_TRY_RC(qvl_dense_ws(st, dt, QVL_EPI_BIAS_GELU, xn, D4, mw.fc1_w, mw.fc1_b, nullptr, 0, h, D4, N / 4, D4, D4,
                            part, L.part_bytes));
  }
  QVL_TRY_RC(qvl_dense_ws(st, dt, QVL_EPI_BIAS, h, D4, mw.fc2_w, mw.fc2_b, nullptr, 0, out, c->out_hidden_size, N / 4,
                          c->out_hidden_size, D4, part, L.part_bytes));
  return QVL_OK;
}

int qvl_encode_vision(void* stream, const qvl_vision_config* c, const qvl_vision_weights* W,
                      const qvl_vision_metadata_dev* meta, const float* px, void* tokens, void* const* deepstack,
                      void* ws, size_t ws_bytes) {
  if (!W || !meta) return set_error(QVL_ERR_INVALID_ARG, "encode_vision: NULL weights/metadata");
  TowerLayout L;
  QVL_TRY_RC(tower_layout(c, meta->n_tokens, &L));
  if (!ws || ws_bytes < L.total) return set_error(QVL_ERR_WORKSPACE, "encode_vision: workspace %zu < %zu", ws_bytes, L.total);
  if (!aligned16(ws)) return set_error(QVL_ERR_MISALIGNED, "encode_vision: workspace alignment");
  if (L.N == 0) return QVL_OK;
  if (!px || !tokens || (c->n_deepstack > 0 && !deepstack)) return set_error(QVL_ERR_INVALID_ARG, "encode_vision: NULL io");
  if (!W->blocks || (c->n_deepstack > 0 && !W->deepstack)) return set_error(QVL_ERR_INVALID_ARG, "encode_vision: NULL weight arrays");
  hipStream_t st = (hipStream_t)stream;
  const int dt = L.dtype;
  const bool f32 = dt == QVL_DTYPE_F32;
  char* base = (char*)ws;
  char* x = base + L.off_x;
  char* xn = base + L.off_xn;
  char* Qb = base + L.off_q;
  char* Kb = base + L.off_k;
  char* Vb = base + L.off_vt;
  char* h = base + L.off_h;
  f32x2* cs = (f32x2*)(base + L.off_cs);
  void* part = L.part_bytes ? base + L.off_part : nullptr;
  float* stats = f32 ? nullptr : (float*)(base + L.off_stats);
  const size_t PB = L.part_bytes;
  const int64_t N = L.N, D = L.D, I = L.I_pad;
  const size_t e = L.esz;
  const float qscale = (1.0f / sqrtf((float)L.hd)) * kLog2e;
  const bool win = c->use_window != 0;
  const int64_t Dout = c->out_hidden_size;
  if (win) {
    if (c->depth > 64) return set_error(QVL_ERR_UNSUPPORTED, "encode_vision: window mode with depth > 64");
    if (!meta->window_index || !meta->window_reverse || (meta->n_window_tiles > 0 && !meta->window_tiles))
      return set_error(QVL_ERR_INVALID_ARG, "encode_vision: window metadata missing");
    // merger outputs are staged in the (then idle) q buffer before the unshuffle
    if ((N / 4) * Dout > L.H * L.Np * L.hdp)
      return set_error(QVL_ERR_UNSUPPORTED, "encode_vision: window mode with out_hidden_size > 4 * hidden");
  }

  // patch embed + learned pos-embed (model.py:802-806), rotary table (807, 821-823); in fp32 the
  // pixels feed the GEMM directly when their rows are a multiple of 64 wide (else they are copied
  // zero-padded, as the bf16 cast is). Window mode: the pixel rows are taken in window order (the
  // reference shuffles x after the row-wise patch embed and pos-embed add, model.py:809-812; the
  // metadata's taps and rotary ids arrive in window order).
  const void* px_in = px;
  if (win) {
    QVL_TRY_RC(gather_rows_pad(st, QVL_DTYPE_F32, px, L.PV, dt, h, L.PVp, meta->window_index, N, 4, L.PV, L.PVp));
    px_in = h;
  } else if (L.PVp != L.PV) {
    QVL_TRY_RC(gather_rows_pad(st, QVL_DTYPE_F32, px, L.PV, dt, h, L.PVp, nullptr, N, 1, L.PV, L.PVp));
    px_in = h;
  } else if (!f32) {
    QVL_TRY_RC(qvl_cast(st, QVL_DTYPE_BF16, px, h, N * L.PV));
    px_in = h;
  }
  // rotary (cos, sin): per token (the relayout kernels, the fp32 path, the head_dim-72 epilogue), or
  // per rotary position for the head_dim-64 fused qkv epilogue when the grid's positions fit its
  // LDS table (measured on MI355X at config 2: 126.6 vs 127.9 us per qkv launch; at head_dim 72
  // the table's 4-byte LDS reads were slower than the per-token loads, 89.3 vs 86.5 us)
  const bool fused_qkv = fused_qkv_rotary(dt, (int)L.hd, (int)L.H);
  // (the folded-LayerNorm qkv kernels leave the table 2 KB less: when any block's qkv Dense carries
  // a fold, the table must fit that smaller limit, since every block reads the one table)
  bool qkv_fold = false;
  for (int i = 0; i < c->depth && !f32; ++i) qkv_fold = qkv_fold || (W->blocks[i].qkv_ln.w && W->blocks[i].qkv_ln.cd);
  const bool pos_tab = fused_qkv && L.hd == 64 && meta->n_positions > 0 &&
                       meta->n_positions * (L.hd / 4) * 4 <= rope_table_lds_bytes((int)L.hd, qkv_fold);
  if (pos_tab)
    QVL_TRY_RC(qvl_rotary_pos_table(st, (int)L.hd, c->rope_theta, (int)meta->n_positions, (uint32_t*)cs));
  else
    QVL_TRY_RC(qvl_rotary_table(st, dt, meta->pos_hw, N, (int)L.hd, c->rope_theta, cs));
  // Folded LayerNorms (bf16 blocks / deepstack mergers whose weights carry the folds) read the row
  // statistics of x as 128-column partials that the residual epilogues writing x (patch embed,
  // proj, fc2) produce beside it: no LayerNorm or statistics launch. have_parts: `stats` holds
  // them for the current x; otherwise a folded LayerNorm runs qvl_row_stats first.
  bool any_fold = false;
  for (int i = 0; i < c->depth && !f32; ++i)
    any_fold = any_fold || (W->blocks[i].qkv_ln.w && W->blocks[i].qkv_ln.cd);
  for (int j = 0; j < c->n_deepstack && !f32; ++j) any_fold = any_fold || W->deepstack[j].fc1_ln.w;
  const int G = any_fold ? L.stat_groups : 0;
  bool have_parts = false;
  if (c->num_position_embeddings > 0 && !f32 && D % 8 == 0) {
    // bf16: the pos-embed gathered per row inside the patch embed's residual epilogue (no [N, D]
    // pos-embed buffer written and read back), with x's row partials when a fold reads them
    QVL_TRY_RC(qvl_dense_pos_embed_ws(st, dt, px_in, L.PVp, W->patch_w, W->patch_b, W->pos_table, meta->tap_idx,
                                      meta->tap_w, x, D, N, D, L.PVp, G ? stats : nullptr, part, PB));
    have_parts = G != 0;
  } else if (c->num_position_embeddings > 0) {
    QVL_TRY_RC(qvl_pos_embed(st, dt, W->pos_table, meta->tap_idx, meta->tap_w, xn, N, D));
    if (G) {
      QVL_TRY_RC(qvl_dense_rowstats_ws(st, dt, px_in, L.PVp, W->patch_w, W->patch_b, xn, D, x, D, N, D, L.PVp, stats,
                                       part, PB));
      have_parts = true;
    } else {
      QVL_TRY_RC(qvl_dense_ws(st, dt, QVL_EPI_BIAS_RESIDUAL, px_in, L.PVp, W->patch_w, W->patch_b, xn, D, x, D, N, D,
                              L.PVp, part, PB));
    }
  } else {   // no learned pos-embed table (model.py:676-680, 803-806): the patch embed alone
    QVL_TRY_RC(qvl_dense_ws(st, dt, QVL_EPI_BIAS, px_in, L.PVp, W->patch_w, W->patch_b, nullptr, 0, x, D, N, D, L.PVp,
                            part, PB));
  }

  int ds_next = 0;
  for (int i = 0; i < c->depth; ++i) {
    const qvl_block_weights& B = W->blocks[i];
    // bf16: norm1 / norm2 folded into the qkv / fc1 GEMMs (the Dense reads x itself; only the row
    // statistics run before it)
    const bool fold = !f32 && B.qkv_ln.w && B.qkv_ln.cd && B.fc1_ln.w && B.fc1_ln.cd;
    // x += proj(attention(rotary(qkv(LN1 x))))   (model.py:628, 569-601)
    if (fold) {
      if (!have_parts) QVL_TRY_RC(qvl_row_stats(st, dt, x, D, N, D, c->ln_eps, stats));
    } else {
      QVL_TRY_RC(qvl_layer_norm(st, dt, x, D, B.norm1_w, B.norm1_b, xn, D, N, D, c->ln_eps));
    }
    if (fused_qkv && fold) {
      const void* tcs = pos_tab ? nullptr : (const void*)cs;
      const int32_t* tpos = pos_tab ? meta->pos_hw : nullptr;
      const uint32_t* ttab = pos_tab ? (const uint32_t*)cs : nullptr;
      const int tnp = pos_tab ? (int)meta->n_positions : 0;
      if (have_parts)
        QVL_TRY_RC(qvl_dense_qkv_rotary_ln_parts(st, dt, x, D, B.qkv_ln.w, B.qkv_ln.cd, stats, G, c->ln_eps, B.qkv_b,
                                                 tcs, tpos, ttab, tnp, Qb, Kb, Vb, N, D, (int)L.H, part, PB));
      else
        QVL_TRY_RC(qvl_dense_qkv_rotary_ln(st, dt, x, D, B.qkv_ln.w, B.qkv_ln.cd, stats, B.qkv_b, tcs, tpos, ttab, tnp,
                                           Qb, Kb, Vb, N, D, (int)L.H, part, PB));
    } else if (fused_qkv) {
      // qkv Dense with rotary + head-major relayout fused into its epilogue.
      if (pos_tab)
        QVL_TRY_RC(qvl_dense_qkv_rotary_pos(st, dt, xn, D, B.qkv_w, B.qkv_b, meta->pos_hw, (const uint32_t*)cs,
                                            (int)meta->n_positions, Qb, Kb, Vb, N, D, (int)L.H, part, PB));
      else
        QVL_TRY_RC(qvl_dense_qkv_rotary(st, dt, xn, D, B.qkv_w, B.qkv_b, cs, Qb, Kb, Vb, N, D, (int)L.H, part, PB));
    } else {
      // qkv Dense into h, then rotary + head-major relayout.
      if (fold && have_parts)
        QVL_TRY_RC(qvl_dense_ln_parts_ws(st, dt, QVL_EPI_BIAS, x, D, B.qkv_ln.w, B.qkv_ln.cd, stats, G, c->ln_eps,
                                         B.qkv_b, h, 3 * D, N, 3 * D, D, part, PB));
      else if (fold)
        QVL_TRY_RC(qvl_dense_ln_ws(st, dt, QVL_EPI_BIAS, x, D, B.qkv_ln.w, B.qkv_ln.cd, stats, B.qkv_b, h, 3 * D, N,
                                   3 * D, D, part, PB));
      else
        QVL_TRY_RC(qvl_dense_ws(st, dt, QVL_EPI_BIAS, xn, D, B.qkv_w, B.qkv_b, nullptr, 0, h, 3 * D, N, 3 * D, D, part,
                                PB));
      if (f32)
        QVL_TRY_RC(attention_relayout_f32((const float*)h, (const float*)h + D, (const float*)h + 2 * D, 3 * D, cs,
                                          (int)N, (int)L.Np, (int)L.H, (int)L.hd, L.vrows, qscale, (float*)Qb,
                                          (float*)Kb, (float*)Vb, st));
      else
        QVL_TRY_RC(attention_relayout_general((const bf16*)h, (const bf16*)h + D, (const bf16*)h + 2 * D, 3 * D, cs,
                                              (int)N, (int)L.Np, (int)L.H, (int)L.hd, L.hdp, L.vrows, qscale,
                                              (bf16*)Qb, (bf16*)Kb, (bf16*)Vb, st));
    }
    // window mode: blocks outside fullatt_block_indexes attend within windows (model.py:838-839)
    const bool full = !win || ((c->fullatt_mask >> i) & 1ull);
    if (full && meta->split_tiles) {
      void* apart = base + L.off_apart;
      QVL_TRY_RC(qvl_attention_headmajor_split(st, dt, Qb, Kb, Vb, meta->split_tiles, meta->n_split_tiles,
                                               meta->n_split_whole, N, (int)L.H, (int)L.hd, xn, D, apart,
                                               L.apart_bytes));
    } else {
      QVL_TRY_RC(qvl_attention_headmajor(st, dt, Qb, Kb, Vb, full ? meta->tiles : meta->window_tiles,
                                         full ? meta->n_tiles : meta->n_window_tiles, N, (int)L.H, (int)L.hd, xn, D));
    }
    have_parts = fold && G;
    if (have_parts)
      QVL_TRY_RC(qvl_dense_rowstats_ws(st, dt, xn, D, B.proj_w, B.proj_b, x, D, x, D, N, D, D, stats, part, PB));
    else
      QVL_TRY_RC(qvl_dense_ws(st, dt, QVL_EPI_BIAS_RESIDUAL, xn, D, B.proj_w, B.proj_b, x, D, x, D, N, D, D, part, PB));
    // x += fc2(gelu(fc1(LN2 x)))   (model.py:629, 610-614)
    if (fold && have_parts) {
      QVL_TRY_RC(qvl_dense_ln_parts_ws(st, dt, QVL_EPI_BIAS_GELU, x, D, B.fc1_ln.w, B.fc1_ln.cd, stats, G, c->ln_eps,
                                       B.fc1_b, h, I, N, I, D, part, PB));
    } else if (fold) {
      QVL_TRY_RC(qvl_row_stats(st, dt, x, D, N, D, c->ln_eps, stats));
      QVL_TRY_RC(qvl_dense_ln_ws(st, dt, QVL_EPI_BIAS_GELU, x, D, B.fc1_ln.w, B.fc1_ln.cd, stats, B.fc1_b, h, I, N, I,
                                 D, part, PB));
    } else {
      QVL_TRY_RC(qvl_layer_norm(st, dt, x, D, B.norm2_w, B.norm2_b, xn, D, N, D, c->ln_eps));
      QVL_TRY_RC(qvl_dense_ws(st, dt, QVL_EPI_BIAS_GELU, xn, D, B.fc1_w, B.fc1_b, nullptr, 0, h, I, N, I, D, part, PB));
    }
    // partials of the new x for the next block's folded norm1 or a folded deepstack merger
    have_parts = G != 0;
    if (have_parts)
      QVL_TRY_RC(qvl_dense_rowstats_ws(st, dt, h, I, B.fc2_w, B.fc2_b, x, D, x, D, N, D, I, stats, part, PB));
    else
      QVL_TRY_RC(qvl_dense_ws(st, dt, QVL_EPI_BIAS_RESIDUAL, h, I, B.fc2_w, B.fc2_b, x, D, x, D, N, D, I, part, PB));
    // deepstack tap (model.py:841-843)
    for (int j = 0; j < c->n_deepstack; ++j)
      if (c->deepstack_indexes[j] == i) {
        void* out = win ? (void*)Qb : deepstack[ds_next];
        QVL_TRY_RC(run_merger(st, c, L, W->deepstack[ds_next], true, x, xn, h, out, part, stats,
                              have_parts ? G : 0));
        if (win)   // unshuffle (model.py:845-848)
          QVL_TRY_RC(qvl_gather_rows(st, dt, Qb, Dout, dt, deepstack[ds_next], Dout, meta->window_reverse, N / 4, 1, Dout));
        ++ds_next;
      }
  }
  (void)e;
  QVL_TRY_RC(run_merger(st, c, L, W->merger, false, x, xn, h, win ? (void*)Qb : tokens, part, stats, 0));
  if (win) QVL_TRY_RC(qvl_gather_rows(st, dt, Qb, Dout, dt, tokens, Dout, meta->window_reverse, N / 4, 1, Dout));
  return QVL_OK;
}

}  // extern "C"
