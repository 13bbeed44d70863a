// bf16 MFMA GEMM with fused epilogues for every Dense of the vision tower.
//
//   y[M, N] = epi(x[M, K] . W[N, K]^T + bias)     (nn.Dense: model.py:556, 570, 601, 611-613, 655-656)
//
// Both operands are K-contiguous ("TN"): activations are row-major [tokens, features] and the
// packed weights are the Flax kernel transposed. A workgroup of WM x WN waves computes a BM x BN
// tile (the planner's shapes: 288x256 and 288x128 on 12 waves, three per SIMD; 256x256 and 256x128
// on 8 waves, two per SIMD); each wave owns a (BM/WM) x (BN/WN) sub-tile of
// v_mfma_f32_32x32x16_bf16 blocks.
// The MFMA "A" operand is the weight tile and "B" the activation tile, so each lane's
// accumulator holds one token row and runs of 4 consecutive output features: the epilogue
// stores 8-byte pieces of a row instead of scattered 2-byte elements.
//
// K loop (BK = 64): operands reach LDS by DMA (buffer_load ... lds, no register staging),
// double-buffered with one barrier per K step; the LDS layout is XOR-swizzled for the 16-lane,
// 64-bank fragment reads; fragments are double-buffered across the four 16-deep k-steps and
// interleaved one read per MFMA.
#include <algorithm>
#include <atomic>

#include "qvl_kernels.h"

namespace qvl {

constexpr int kBK = 64;

// Tile of BM x BN outputs per workgroup of WM x WN waves; each wave owns TM x TN = (BM/WM) x
// (BN/WN) built from 32x32 MFMA blocks (MB x NB of them).
template <int BM, int BN, int WM, int WN>
struct GemmShape {
  static constexpr int THREADS = 64 * WM * WN;
  static constexpr int TM = BM / WM, TN = BN / WN;
  static constexpr int MB = TM / 32, NB = TN / 32;
  static constexpr int ROWS_PER_PASS = THREADS / 8;     // rows one DMA pass (8 per wave) covers
  static_assert(BM % 8 == 0 && BN % 8 == 0 && TM % 32 == 0 && TN % 32 == 0, "tile shape");
  // DMA passes per operand; the last pass may cover only part of the waves (predicated per wave).
  static constexpr int XPT = (BM + ROWS_PER_PASS - 1) / ROWS_PER_PASS, WPT = (BN + ROWS_PER_PASS - 1) / ROWS_PER_PASS;
  static constexpr int LDS_ELEMS = (BM + BN) * kBK;    // one stage
};

// LDS element offset of (row, 16-byte chunk). Rows are 128 bytes; the LDS serves a 16-byte read
// for 16 lanes per clock across 64 banks, i.e. two rows' worth, so rows r and r+1 fall in
// different bank halves and the chunk is XOR-swizzled with (r/2) % 8: the 16 consecutive rows a
// fragment read touches in one clock hit 16 distinct 16-byte bank groups.
__device__ __forceinline__ int lds_off(int row, int chunk) {
  return row * kBK + ((chunk ^ ((row >> 1) & 7)) << 3);
}

// ---------------------------------------------------------------------------------------------
// Epilogue pieces, shared by the GEMM and the split-K reduction.
// ---------------------------------------------------------------------------------------------
// The epilogues round at the reference's cast points (flax Dense in bf16, model.py:556-613):
// y = bf16(bf16(x.W) + bias); GELU: bf16(gelu(y)); residual: bf16(res + y).
template <int EPI>
__device__ __forceinline__ float epi_value(float acc, float bias) {
  float v = round_bf16(round_bf16(acc) + bias);
  if constexpr (EPI == kEpiBiasGelu) v = gelu_tanh(v);
  return v;
}

// Bias (+ GELU | + residual) on 4 consecutive features n..n+3 of token m, one bf16 store.
template <int EPI>
__device__ __forceinline__ void epi_store_quad(const GemmParams& p, int m, int n, const float (&acc4)[4]) {
  if (m >= p.M || n >= p.N) return;
  const f32x4 bv = *reinterpret_cast<const f32x4*>(p.bias + n);
  float v[4];
#pragma unroll
  for (int e = 0; e < 4; ++e) v[e] = epi_value<EPI>(acc4[e], bv[e]);
  if constexpr (EPI == kEpiBiasResidual) {
    const u32x2 r = *reinterpret_cast<const u32x2*>(p.res + (int64_t)m * p.ldr + n);
    v[0] += bf16_lo(r.x); v[1] += bf16_hi(r.x); v[2] += bf16_lo(r.y); v[3] += bf16_hi(r.y);
  }
  const u32x2 o = {pack_bf16x2(v[0], v[1]), pack_bf16x2(v[2], v[3])};
  *reinterpret_cast<u32x2*>(p.y + (int64_t)m * p.ldc + n) = o;
}

// Rounds a and b to bf16 (kept as floats) with one packed conversion (round to nearest even).
// Written as the instruction itself: from the C form the compiler splits the pair into two
// single-value conversions, one per half it extracts.
__device__ __forceinline__ void round_bf16_pair(float& a, float& b) {
  uint32_t w;
  asm("v_cvt_pk_bf16_f32 %0, %1, %2" : "=v"(w) : "v"(a), "v"(b));
  a = bf16_lo(w);
  b = bf16_hi(w);
}

// The learned pos-embed of one token at features n..n+7 (model.py:751-764) for kEpiBiasPosEmbed,
// in the arithmetic of the pos-embed kernel: each tap product rounded to bf16, the partial sums
// taken left to right and rounded, taps of weight 0 skipped (their products are zeros). `tap`: the
// token's 4 (index, weight bits) pairs, staged in LDS; every live tap's table row is loaded before
// any is combined.
__device__ __forceinline__ void pos_embed_oct(const GemmParams& p, const int2* tap, int n, float (&acc)[8]) {
  const int4 t01 = *reinterpret_cast<const int4*>(tap), t23 = *reinterpret_cast<const int4*>(tap + 2);
  const int ti[4] = {t01.x, t01.z, t23.x, t23.z};
  const float tw[4] = {__int_as_float(t01.y), __int_as_float(t01.w), __int_as_float(t23.y), __int_as_float(t23.w)};
  u32x4 row[4];
#pragma unroll
  for (int j = 0; j < 4; ++j)
    row[j] = tw[j] != 0.f ? *reinterpret_cast<const u32x4*>(p.pe_table + (int64_t)ti[j] * p.N + n) : u32x4{0u, 0u, 0u, 0u};
  bool first = true;
#pragma unroll
  for (int e = 0; e < 8; ++e) acc[e] = 0.f;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    if (tw[j] == 0.f) continue;
    const u32x4 w = row[j];
    const float v[8] = {bf16_lo(w.x), bf16_hi(w.x), bf16_lo(w.y), bf16_hi(w.y),
                        bf16_lo(w.z), bf16_hi(w.z), bf16_lo(w.w), bf16_hi(w.w)};
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const float t = round_bf16(tw[j] * v[e]);
      acc[e] = first ? t : round_bf16(acc[e] + t);
    }
    first = false;
  }
}

// Same on 8 consecutive features n..n+7 whose products arrive already rounded to bf16 (packed
// pairs, from the LDS-staged tile), with the bias of those features preloaded (b0 | b1, zeros
// past N): 16-byte loads/stores when the rows are 16-byte aligned. The products are exact bf16
// values, so only the sum with the bias is rounded (pairwise, one conversion per two values).
template <int EPI>
__device__ __forceinline__ u32x4 epi_store_oct(const GemmParams& p, int m, int n, u32x4 raw, const f32x4& b0,
                                               const f32x4& b1, bool full, bool vec16, const int2* tap = nullptr) {
  float v[8] = {bf16_lo(raw.x) + b0[0], bf16_hi(raw.x) + b0[1], bf16_lo(raw.y) + b0[2], bf16_hi(raw.y) + b0[3],
                bf16_lo(raw.z) + b1[0], bf16_hi(raw.z) + b1[1], bf16_lo(raw.w) + b1[2], bf16_hi(raw.w) + b1[3]};
  if constexpr (EPI != kEpiBias) {
#pragma unroll
    for (int e = 0; e < 8; e += 2) round_bf16_pair(v[e], v[e + 1]);
  }
  if constexpr (EPI == kEpiBiasGelu) {
#pragma unroll
    for (int e = 0; e < 8; ++e) v[e] = gelu_tanh(v[e]);
  }
  bf16* dst = p.y + (int64_t)m * p.ldc + n;
  if constexpr (EPI == kEpiBiasPosEmbed) {
    // (the host guarantees whole, 16-byte aligned octets for this epilogue)
    float r[8];
    pos_embed_oct(p, tap, n, r);
#pragma unroll
    for (int e = 0; e < 8; ++e) v[e] += r[e];
    const u32x4 o = {pack_bf16x2(v[0], v[1]), pack_bf16x2(v[2], v[3]), pack_bf16x2(v[4], v[5]), pack_bf16x2(v[6], v[7])};
    __builtin_nontemporal_store(o, reinterpret_cast<u32x4*>(dst));
    return o;
  }
  if (vec16 && full) {
    if constexpr (EPI == kEpiBiasResidual) {
      const u32x4 r = *reinterpret_cast<const u32x4*>(p.res + (int64_t)m * p.ldr + n);
      v[0] += bf16_lo(r.x); v[1] += bf16_hi(r.x); v[2] += bf16_lo(r.y); v[3] += bf16_hi(r.y);
      v[4] += bf16_lo(r.z); v[5] += bf16_hi(r.z); v[6] += bf16_lo(r.w); v[7] += bf16_hi(r.w);
    }
    // Streaming (nt) store: every CU writes its whole tile at once at the end of a round, and
    // the output is not re-read by this kernel; measured ~1.5% faster per tower forward.
    const u32x4 o = {pack_bf16x2(v[0], v[1]), pack_bf16x2(v[2], v[3]), pack_bf16x2(v[4], v[5]), pack_bf16x2(v[6], v[7])};
    __builtin_nontemporal_store(o, reinterpret_cast<u32x4*>(dst));
    return o;
  }
  u32x4 o = {0u, 0u, 0u, 0u};
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    if (h == 1 && !full) break;
    if constexpr (EPI == kEpiBiasResidual) {
      const u32x2 r = *reinterpret_cast<const u32x2*>(p.res + (int64_t)m * p.ldr + n + 4 * h);
      v[4 * h] += bf16_lo(r.x); v[4 * h + 1] += bf16_hi(r.x); v[4 * h + 2] += bf16_lo(r.y); v[4 * h + 3] += bf16_hi(r.y);
    }
    const u32x2 oh = {pack_bf16x2(v[4 * h], v[4 * h + 1]), pack_bf16x2(v[4 * h + 2], v[4 * h + 3])};
    *reinterpret_cast<u32x2*>(dst + 4 * h) = oh;
    o[2 * h] = oh.x;
    o[2 * h + 1] = oh.y;
  }
  return o;
}

// Statistics of the LayerNorm that reads this epilogue's output next (p.rs_part): the bf16 values
// w of 8 consecutive columns n..n+7 of row m, one such octet per lane, 16 lanes (aligned to 16)
// holding the 16 octets of one 128-column group; the group's sum and its sum of squared deviations
// from the group mean go to rs_part (two butterfly reductions over the 16 lanes; every lane ends
// with the same bits, IEEE addition being commutative).
__device__ __forceinline__ void row_group_stats(const GemmParams& p, int m, int n, u32x4 w) {
  const float y[8] = {bf16_lo(w.x), bf16_hi(w.x), bf16_lo(w.y), bf16_hi(w.y),
                      bf16_lo(w.z), bf16_hi(w.z), bf16_lo(w.w), bf16_hi(w.w)};
  float s = ((y[0] + y[1]) + (y[2] + y[3])) + ((y[4] + y[5]) + (y[6] + y[7]));
#pragma unroll
  for (int o = 1; o < 16; o <<= 1) s += __shfl_xor(s, o);
  const float mean = s * (1.0f / 128.0f);
  float q = 0.f;
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    const float d = y[e] - mean;
    q = fmaf(d, d, q);
  }
#pragma unroll
  for (int o = 1; o < 16; o <<= 1) q += __shfl_xor(q, o);
  if ((threadIdx.x & 15) == 0) p.rs_part[(int64_t)m * (p.N / 128) + n / 128] = f32x2{s, q};
}

// (mean, rstd) of row m for a folded LayerNorm: from p.ln_stats, or combined from the row's
// 128-column partials (Chan et al.'s pairwise update: M2 = sum_g [Q_g + (S_g - 128 mean)^2 / 128]),
// var = M2 / K, rstd = 1 / sqrt(var + eps) (model.py:384-386). Rows at or past M give zeros.
// A row's partials are loaded kLnChunk at a time (an unrolled, guarded loop: every load of a
// chunk is in flight before the first use) and combined in registers; a row of at most kLnChunk
// groups (the blocks' LayerNorms: hidden / 128) is loaded once for both passes.
constexpr int kLnChunk = 16;

__device__ __forceinline__ f32x2 ln_row(const GemmParams& p, int m) {
  if (m >= p.M) return f32x2{0.f, 0.f};
  if (!p.ln_part) return p.ln_stats[m];
  const int G = p.ln_groups;
  const f32x2* q = p.ln_part + (int64_t)m * G;
  f32x2 v[kLnChunk];
  auto load = [&](int base) {
#pragma unroll
    for (int g = 0; g < kLnChunk; ++g) v[g] = base + g < G ? q[base + g] : f32x2{0.f, 0.f};
  };
  float s = 0.f;
  for (int base = 0; base < G; base += kLnChunk) {
    load(base);
#pragma unroll
    for (int g = 0; g < kLnChunk; ++g) s += v[g].x;
  }
  const float inv_n = 1.0f / (128.0f * (float)G);
  const float mean = s * inv_n;
  float m2 = 0.f;
  for (int base = 0; base < G; base += kLnChunk) {
    if (G > kLnChunk) load(base);
#pragma unroll
    for (int g = 0; g < kLnChunk; ++g) {
      const float d = v[g].x - 128.0f * mean;
      if (base + g < G) m2 += v[g].y + d * d * (1.0f / 128.0f);
    }
  }
  return f32x2{mean, rsqrtf(m2 * inv_n + p.ln_eps)};
}

__device__ __forceinline__ void rope_values(const GemmParams& p, int which, int m, int d, const f32x4& blo,
                                            const f32x4& bhi, const float (&lo_acc)[4], const float (&hi_acc)[4],
                                            const f32x4& c01, const f32x4& c23, u32x2& o1, u32x2& o2);

// Folded LayerNorm (p.ln_stats or p.ln_part): the 4 accumulators of features n..n+3 of token m become
// rstd * acc - rstd * mean * c + d, i.e. LN(x) . W (model.py:387 into 556), before any rounding.
__device__ __forceinline__ void ln_fold_quad(const GemmParams& p, int m, int n, float (&a)[4]) {
  const f32x2 st = ln_row(p, m);
  const f32x4 cd01 = *reinterpret_cast<const f32x4*>(p.ln_cd + n), cd23 = *reinterpret_cast<const f32x4*>(p.ln_cd + n + 2);
  const float nm = -st.x * st.y;
  a[0] = fmaf(a[0], st.y, fmaf(nm, cd01[0], cd01[1]));
  a[1] = fmaf(a[1], st.y, fmaf(nm, cd01[2], cd01[3]));
  a[2] = fmaf(a[2], st.y, fmaf(nm, cd23[0], cd23[1]));
  a[3] = fmaf(a[3], st.y, fmaf(nm, cd23[2], cd23[3]));
}

// The fold on a workgroup's accumulators, applied where each epilogue reads them (acc[a][b][4 g + e]
// is token m0 + wm TM + 32 b + l32, feature n0 + wn TN + 32 a + 8 g + 4 hh + e): the rows'
// (rstd, -mean * rstd) are loaded once, then each 4-feature group takes its (c, d) from the LDS
// copy as it is staged.
template <int MB>
struct LnRows {
  float r[MB], nm[MB];
};

// lrs: the tile's rows' (rstd, -mean * rstd) in LDS (row m0 + i at lrs[i]), r_first: the lane's first row.
template <int MB>
__device__ __forceinline__ LnRows<MB> ln_rows(const f32x2* lrs, int r_first) {
  LnRows<MB> L;
#pragma unroll
  for (int b = 0; b < MB; ++b) {
    const f32x2 v = lrs[r_first + 32 * b];
    L.r[b] = v.x;
    L.nm[b] = v.y;
  }
  return L;
}

// lcd: the tile's (c, d) pairs in LDS (column n0 + i at lcd[i], zeros past N), copied at kernel start.
__device__ __forceinline__ void ln_fold_cd(const f32x4& cd01, const f32x4& cd23, float r, float nm, float (&v)[4]) {
  v[0] = fmaf(v[0], r, fmaf(nm, cd01[0], cd01[1]));
  v[1] = fmaf(v[1], r, fmaf(nm, cd01[2], cd01[3]));
  v[2] = fmaf(v[2], r, fmaf(nm, cd23[0], cd23[1]));
  v[3] = fmaf(v[3], r, fmaf(nm, cd23[2], cd23[3]));
}

__device__ __forceinline__ void ln_fold_group(const f32x2* lcd, float r, float nm, int col, float (&v)[4]) {
  ln_fold_cd(*reinterpret_cast<const f32x4*>(lcd + col), *reinterpret_cast<const f32x4*>(lcd + col + 2), r, nm, v);
}


// (cos, sin) of the 4 dims d..d+3 (< head_dim/2) of token m as (c_d, s_d, c_d+1, s_d+1) |
// (c_d+2, s_d+2, c_d+3, s_d+3): from the per-token table p.cs, or from the per-position table
// p.rtab (global memory) at the token's (h, w) ids. Tokens past M get anything (their outputs are
// zeros).
__device__ __forceinline__ void unpack_cs4(const uint32_t (&w)[4], f32x4& c01, f32x4& c23) {
  c01 = f32x4{bf16_lo(w[0]), bf16_hi(w[0]), bf16_lo(w[1]), bf16_hi(w[1])};
  c23 = f32x4{bf16_lo(w[2]), bf16_hi(w[2]), bf16_lo(w[3]), bf16_hi(w[3])};
}

template <typename T>
__device__ __forceinline__ void rope_cs_table(const T* tab, int q4, int ph, int pw, int d, f32x4& c01, f32x4& c23) {
  uint32_t w[4];
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    const int j = d + e;
    w[e] = j < q4 ? tab[ph * q4 + j] : tab[pw * q4 + j - q4];
  }
  unpack_cs4(w, c01, c23);
}

__device__ __forceinline__ void token_pos(const GemmParams& p, int m, int& ph, int& pw) {
  ph = 0;
  pw = 0;
  if (m < p.M) {
    ph = min(max(p.pos_hw[2 * m], 0), p.rtab_pos - 1);     // clamped: table lookups stay in bounds
    pw = min(max(p.pos_hw[2 * m + 1], 0), p.rtab_pos - 1);
  }
}

__device__ __forceinline__ void rope_cs_global(const GemmParams& p, int m, int d, f32x4& c01, f32x4& c23) {
  if (p.rtab) {
    int ph, pw;
    token_pos(p, m, ph, pw);
    rope_cs_table(p.rtab, p.cs_half / 2, ph, pw, d, c01, c23);
    return;
  }
  if (m >= p.M) { c01 = f32x4{}; c23 = f32x4{}; return; }
  const f32x4* csr = reinterpret_cast<const f32x4*>(p.cs + (int64_t)m * p.cs_half + d);
  c01 = csr[0];
  c23 = csr[1];
}

// Rotary epilogue of the qkv GEMM for one pair of quads (the split-K reduction's path): features
// n..n+3 (dims d..d+3 < 32 of a head) and n+32..n+35 of token m, stored straight to q/k
// [H][Np][64] and v^T [H][64][Np] at key position vt_pos(m). Tokens in [M, Np) get zeros.
__device__ __forceinline__ void epi_rope_pair(const GemmParams& p, int m, int n, const float (&lo_acc)[4],
                                              const float (&hi_acc)[4]) {
  if (m >= p.Np || n >= p.N) return;
  const int which = n / p.D;                 // 0 = q, 1 = k, 2 = v
  const int head = (n % p.D) / 64, d = n % 64;
  const f32x4 blo = *reinterpret_cast<const f32x4*>(p.bias + n);
  const f32x4 bhi = *reinterpret_cast<const f32x4*>(p.bias + n + 32);
  u32x2 o1, o2;
  f32x4 c01 = {}, c23 = {};
  if (which < 2) rope_cs_global(p, m, d, c01, c23);
  rope_values(p, which, m, d, blo, bhi, lo_acc, hi_acc, c01, c23, o1, o2);
  if (which == 2) {
    bf16* vt = p.vt + (int64_t)head * 64 * p.Np + vt_pos(m);
    const uint32_t w[4] = {o1.x, o1.y, o2.x, o2.y};
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      vt[(int64_t)(d + e) * p.Np] = __builtin_bit_cast(bf16, (uint16_t)(w[e >> 1] >> (16 * (e & 1))));
      vt[(int64_t)(d + e + 32) * p.Np] = __builtin_bit_cast(bf16, (uint16_t)(w[2 + (e >> 1)] >> (16 * (e & 1))));
    }
    return;
  }
  bf16* dst = (which == 0 ? p.q : p.k) + ((int64_t)head * p.Np + m) * 64;
  *reinterpret_cast<u32x2*>(dst + d) = o1;
  *reinterpret_cast<u32x2*>(dst + d + 32) = o2;
}

// LDS-staged epilogue: each wave writes bf16(acc) of its sub-tile into the (free) LDS as a
// row-major BM x BN tile whose 16-byte chunks are XOR-swizzled by row (chunk ^ row % (BN/8)),
// so the 32 rows one ds_write_b64 touches land on distinct chunks; then the workgroup walks the
// tile row by row, 16 bytes (8 features) per lane, and applies bias / GELU / residual with whole
// rows per load and store instead of 8-byte pieces of 32 rows.
template <int BM, int BN, int WM, int WN, int EPI, bool LN>
__device__ __forceinline__ void gemm_epilogue_lds(const GemmParams& p,
                                                  f32x16 (&acc)[GemmShape<BM, BN, WM, WN>::NB][GemmShape<BM, BN, WM, WN>::MB],
                                                  int m0, int n0, int wm, int wn, int lane, int tid, bf16* smem,
                                                  const f32x2* lcd, const int2* ltaps) {
  using S = GemmShape<BM, BN, WM, WN>;
  constexpr int CH = BN / 8;
  const int l32 = lane & 31, hh = lane >> 5;
  LnRows<S::MB> L;
  if constexpr (LN) L = ln_rows<S::MB>(lcd + BN, wm * S::TM + l32);
  // (column groups outermost: a folded LayerNorm's (c, d) of a lane's 4 columns are read once for
  // all its row blocks)
#pragma unroll
  for (int a = 0; a < S::NB; ++a)
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      const int c = (wn * S::TN + a * 32) / 8 + g;
      f32x4 cd01 = {}, cd23 = {};
      if constexpr (LN) {
        cd01 = *reinterpret_cast<const f32x4*>(lcd + c * 8 + 4 * hh);
        cd23 = *reinterpret_cast<const f32x4*>(lcd + c * 8 + 4 * hh + 2);
      }
#pragma unroll
      for (int b = 0; b < S::MB; ++b) {
        const int r = wm * S::TM + b * 32 + l32;
        float f[4] = {acc[a][b][4 * g], acc[a][b][4 * g + 1], acc[a][b][4 * g + 2], acc[a][b][4 * g + 3]};
        if constexpr (LN) ln_fold_cd(cd01, cd23, L.r[b], L.nm[b], f);
        const u32x2 v = {pack_bf16x2(f[0], f[1]), pack_bf16x2(f[2], f[3])};
        *reinterpret_cast<u32x2*>(smem + r * BN + ((c ^ (r % CH)) << 3) + hh * 4) = v;
      }
    }
  __syncthreads();
  const bool vec16 = ((p.ldc | (EPI == kEpiBiasResidual ? p.ldr : 0)) & 7) == 0;
  // A thread keeps one 8-feature column group for the whole walk (THREADS is a multiple of the
  // groups per row), so its bias is loaded once.
  static_assert(S::THREADS % CH == 0 && BM % (S::THREADS / CH) == 0, "epilogue walk");
  constexpr int RSTEP = S::THREADS / CH;
  const int c = tid % CH, n = n0 + c * 8;
  if (n >= p.N) return;
  const bool full = n + 8 <= p.N;
  const f32x4 b0 = *reinterpret_cast<const f32x4*>(p.bias + n);
  const f32x4 b1 = full ? *reinterpret_cast<const f32x4*>(p.bias + n + 4) : f32x4{};
#pragma unroll 4
  for (int i = 0; i < BM / RSTEP; ++i) {
    const int r = i * RSTEP + tid / CH;
    const int m = m0 + r;
    if (m >= p.M) break;               // rows only grow with i
    const u32x4 raw = *reinterpret_cast<const u32x4*>(smem + r * BN + ((c ^ (r % CH)) << 3));
    const u32x4 out = epi_store_oct<EPI>(p, m, n, raw, b0, b1, full, vec16, ltaps ? ltaps + 4 * r : nullptr);
    if constexpr (EPI == kEpiBiasResidual || EPI == kEpiBiasPosEmbed) {
      // 16 consecutive threads, aligned to 16, hold the 16 octets of one 128-column group of row m
      static_assert(CH % 16 == 0, "row statistics need 128-column groups within a tile row");
      if (p.rs_part) row_group_stats(p, m, n, out);
    }
  }
}

// Rotary qkv values of 4 consecutive dims d..d+3 (< 32) and d+32..d+35 of one head, for token m,
// as packed bf16 pairs: bias (blo = bias[n..n+3], bhi = bias[n+32..n+35]), the reference's bf16
// cast points, rotary (q, k) and the softmax pre-scale (q). Tokens at or past M give zeros (the
// attention kernel's padding). Every rounding is the reference's; pairs of them share one
// packed conversion.
__device__ __forceinline__ void rope_values(const GemmParams& p, int which, int m, int d, const f32x4& blo,
                                            const f32x4& bhi, const float (&lo_acc)[4], const float (&hi_acc)[4],
                                            const f32x4& c01, const f32x4& c23, u32x2& o1, u32x2& o2) {
  if (m >= p.M) {
    o1 = u32x2{0u, 0u};
    o2 = u32x2{0u, 0u};
    return;
  }
  float lo[4] = {lo_acc[0], lo_acc[1], lo_acc[2], lo_acc[3]};
  float hi[4] = {hi_acc[0], hi_acc[1], hi_acc[2], hi_acc[3]};
#pragma unroll
  for (int e = 0; e < 4; e += 2) { round_bf16_pair(lo[e], lo[e + 1]); round_bf16_pair(hi[e], hi[e + 1]); }
#pragma unroll
  for (int e = 0; e < 4; ++e) { lo[e] += blo[e]; hi[e] += bhi[e]; }
  if (which == 2) {
    o1 = u32x2{pack_bf16x2(lo[0], lo[1]), pack_bf16x2(lo[2], lo[3])};
    o2 = u32x2{pack_bf16x2(hi[0], hi[1]), pack_bf16x2(hi[2], hi[3])};
    return;
  }
#pragma unroll
  for (int e = 0; e < 4; e += 2) { round_bf16_pair(lo[e], lo[e + 1]); round_bf16_pair(hi[e], hi[e + 1]); }
  const float cs_c[4] = {c01[0], c01[2], c23[0], c23[2]};
  const float cs_s[4] = {c01[1], c01[3], c23[1], c23[3]};
  // x*cos + rotate_half(x)*sin with each product and the sum rounded (model.py:579-582):
  // dims < hd/2: lo*cos - hi*sin; dims + hd/2: hi*cos + lo*sin.
  float lc[4], hs[4], hc[4], ls[4];
#pragma unroll
  for (int e = 0; e < 4; ++e) { lc[e] = lo[e] * cs_c[e]; hs[e] = hi[e] * cs_s[e]; hc[e] = hi[e] * cs_c[e]; ls[e] = lo[e] * cs_s[e]; }
#pragma unroll
  for (int e = 0; e < 4; e += 2) {
    round_bf16_pair(lc[e], lc[e + 1]); round_bf16_pair(hs[e], hs[e + 1]);
    round_bf16_pair(hc[e], hc[e + 1]); round_bf16_pair(ls[e], ls[e + 1]);
  }
  float r1[4], r2[4];
#pragma unroll
  for (int e = 0; e < 4; ++e) { r1[e] = lc[e] - hs[e]; r2[e] = hc[e] + ls[e]; }
  if (which == 0) {                             // q: round the sum, then the pre-scale
#pragma unroll
    for (int e = 0; e < 4; e += 2) { round_bf16_pair(r1[e], r1[e + 1]); round_bf16_pair(r2[e], r2[e + 1]); }
#pragma unroll
    for (int e = 0; e < 4; ++e) { r1[e] *= p.qscale; r2[e] *= p.qscale; }
  }
  o1 = u32x2{pack_bf16x2(r1[0], r1[1]), pack_bf16x2(r1[2], r1[3])};
  o2 = u32x2{pack_bf16x2(r2[0], r2[1]), pack_bf16x2(r2[2], r2[3])};
}

// LDS-staged rotary epilogue of the qkv GEMM. A wave's TN features are whole heads of one of q,
// k, v; it writes its TM x TN block of final bf16 values into its own LDS region (row-major,
// 16-byte chunks XOR-swizzled by row), then streams it out: q/k rows of a head are 128 contiguous
// bytes of [H][Np][64] (16 bytes per lane), and v goes out transposed to [H][64][Np] as 16-byte
// runs of 8 key positions (gathered from the block with the vt_pos quad swap), instead of
// 8-byte pieces of 32 rows (q, k) and 2-byte scattered stores (v).
template <int BM, int BN, int WM, int WN, bool LN>
__device__ __forceinline__ void gemm_epilogue_rope_lds(const GemmParams& p,
                                                       f32x16 (&acc)[GemmShape<BM, BN, WM, WN>::NB][GemmShape<BM, BN, WM, WN>::MB],
                                                       int m0, int n0, int wm, int wn, int lane, int wave, bf16* smem,
                                                       const uint32_t* ltab, const f32x2* lcd) {
  using S = GemmShape<BM, BN, WM, WN>;
  constexpr int TM = S::TM, TN = S::TN, CPR = TN / 8, HPW = TN / 64;
  static_assert(TN % 64 == 0 && TM % 16 == 0, "the rotary epilogue needs whole heads and 16-token groups");
  constexpr int RSH = TN == 64 ? 1 : 0;          // rows per 256-byte bank row: 2 (TN 64) or 1 (TN 128)
  bf16* reg = smem + wave * TM * TN;
  auto off = [](int row, int chunk) { return row * TN + ((chunk ^ ((row >> RSH) & (CPR - 1))) << 3); };
  const int l32 = lane & 31, hh = lane >> 5;
  const int nw = n0 + wn * TN;                   // first feature of the wave's block
  if (nw >= p.N) return;
  const int which = nw / p.D;                    // 0 = q, 1 = k, 2 = v
  const int head0 = (nw % p.D) / 64;
  const int base = m0 + wm * TM;                 // first token of the wave's block
  // rotary (h, w) ids of the lane's tokens, for the LDS position table
  int ph[S::MB], pw[S::MB];
  if (ltab && which < 2) {
#pragma unroll
    for (int b = 0; b < S::MB; ++b) token_pos(p, base + b * 32 + l32, ph[b], pw[b]);
  }
  // one (head, 4 dims, token block) unit: bias, the folded LayerNorm (LN: the token's (rstd,
  // -mean * rstd) from the LDS copy, read where the unit needs it), rotary, into LDS
  auto unit = [&](int h2, int g, int b, const f32x4& blo, const f32x4& bhi) {
    const int d = 8 * g + 4 * hh, n = nw + h2 * 64 + d;
    const int t = b * 32 + l32;
    float lo[4], hi[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) { lo[e] = acc[2 * h2][b][4 * g + e]; hi[e] = acc[2 * h2 + 1][b][4 * g + e]; }
    if constexpr (LN) {
      const f32x2 rs = lcd[BN + wm * S::TM + t];
      ln_fold_group(lcd, rs.x, rs.y, n - n0, lo);
      ln_fold_group(lcd, rs.x, rs.y, n - n0 + 32, hi);
    }
    f32x4 c01 = {}, c23 = {};
    if (which < 2) {
      if (ltab) {
        // dims d..d+3 lie in one half (d % 4 == 0, head_dim / 4 = 16): one 16-byte LDS read
        uint32_t w[4];
        const u32x4 q = *reinterpret_cast<const u32x4*>(ltab + (d < 16 ? ph[b] : pw[b]) * 16 + (d & 15));
        w[0] = q.x; w[1] = q.y; w[2] = q.z; w[3] = q.w;
        unpack_cs4(w, c01, c23);
      } else {
        rope_cs_global(p, base + t, d, c01, c23);
      }
    }
    u32x2 o1, o2;
    rope_values(p, which, base + t, d, blo, bhi, lo, hi, c01, c23, o1, o2);
    *reinterpret_cast<u32x2*>(reg + off(t, h2 * 8 + g) + 4 * hh) = o1;
    *reinterpret_cast<u32x2*>(reg + off(t, h2 * 8 + 4 + g) + 4 * hh) = o2;
  };
  auto bias_of = [&](int h2, int g, f32x4& blo, f32x4& bhi) {
    const int n = nw + h2 * 64 + 8 * g + 4 * hh;
    blo = *reinterpret_cast<const f32x4*>(p.bias + n);
    bhi = *reinterpret_cast<const f32x4*>(p.bias + n + 32);
  };
  if constexpr (LN) {
    // token blocks outermost: a unit's (c, d) and bias are used once, so none stay live across
    // units beside the accumulators
#pragma unroll
    for (int b = 0; b < S::MB; ++b)
#pragma unroll
      for (int h2 = 0; h2 < HPW; ++h2)
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          f32x4 blo, bhi;
          bias_of(h2, g, blo, bhi);
          unit(h2, g, b, blo, bhi);
          __builtin_amdgcn_sched_barrier(0);
        }
  } else {
#pragma unroll
    for (int h2 = 0; h2 < HPW; ++h2)
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        f32x4 blo, bhi;
        bias_of(h2, g, blo, bhi);                 // once per (head, dims)
#pragma unroll
        for (int b = 0; b < S::MB; ++b) unit(h2, g, b, blo, bhi);
      }
  }
  // (a wave reads back only its own region; its LDS operations complete in order)
  if (which < 2) {
    bf16* dst = which == 0 ? p.q : p.k;
    constexpr int RPI = 64 / CPR;                 // rows per instruction
#pragma unroll 4
    for (int i = 0; i < TM / RPI; ++i) {
      const int t = i * RPI + lane / CPR, c = lane % CPR;
      const int m = base + t;
      const u32x4 v = *reinterpret_cast<const u32x4*>(reg + off(t, c));
      if (m < p.Np) *reinterpret_cast<u32x4*>(dst + ((int64_t)(head0 + c / 8) * p.Np + m) * 64 + (c % 8) * 8) = v;
    }
  } else {
    // One lane per (head, 4 dims, 8 positions): 8 reads of 4 dims of a token, regrouped by
    // v_perm into the 4 rows' 16-byte runs.
    constexpr int PCH = TM / 8;                   // 8-position chunks per V^T row
    constexpr int ITEMS = HPW * 16 * PCH;
    static_assert(ITEMS % 64 == 0, "V^T work items must fill whole waves");
#pragma unroll 1
    for (int i = 0; i < ITEMS / 64; ++i) {
      const int item = i * 64 + lane;
      const int r = item / PCH, pc = item % PCH;  // r: head-in-wave * 16 + dim quad
      const int h2 = r / 16, d = (r % 16) * 4;
      const int P = base + pc * 8;                // 8 consecutive V^T positions
      uint32_t w01[8], w23[8];                    // dims (d, d+1) and (d+2, d+3) at position P + e
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const int t = vt_pos(P + e) - base;       // the token stored at position P + e
        const u32x2 v = *reinterpret_cast<const u32x2*>(reg + off(t, h2 * 8 + d / 8) + (d & 7));
        w01[e] = v.x;
        w23[e] = v.y;
      }
      if (P < p.Np) {
        bf16* row = p.vt + ((int64_t)(head0 + h2) * 64 + d) * p.Np + P;
        u32x4 o0, o1, o2, o3;
#pragma unroll
        for (int k = 0; k < 4; ++k) {
          o0[k] = __builtin_amdgcn_perm(w01[2 * k + 1], w01[2 * k], 0x05040100u);   // low halves: dim d
          o1[k] = __builtin_amdgcn_perm(w01[2 * k + 1], w01[2 * k], 0x07060302u);   // high halves: dim d+1
          o2[k] = __builtin_amdgcn_perm(w23[2 * k + 1], w23[2 * k], 0x05040100u);
          o3[k] = __builtin_amdgcn_perm(w23[2 * k + 1], w23[2 * k], 0x07060302u);
        }
        *reinterpret_cast<u32x4*>(row) = o0;
        *reinterpret_cast<u32x4*>(row + p.Np) = o1;
        *reinterpret_cast<u32x4*>(row + 2 * (int64_t)p.Np) = o2;
        *reinterpret_cast<u32x4*>(row + 3 * (int64_t)p.Np) = o3;
      }
    }
  }
}

// Rotary epilogue of the head_dim-72 qkv GEMM (tile 256 x 288 = 4 whole heads of one of q, k, v):
// the waves stage bf16(acc) in the (free) LDS as a row-major 256 x 288 tile (row stride kR72),
// then the workgroup walks it. q / k: items (token, head, 4 rotary pairs), each the 4 dims d..d+3
// and d+36..d+39 through rope_values (bias, the reference's roundings, the q pre-scale), stored
// to rows of 88 dims [H][Np][88] whose dims 72..87 are zero. v: items (head, 2 dims, 8 key
// positions), 8 LDS reads of one token's pair each, stored as two 16-byte runs of V^T [H][72][Np]
// at the vt_pos positions. Tokens in [M, Np) get zeros.
constexpr int kR72 = 296;   // LDS row stride (elements) of the staged tile: 592 bytes, 16-byte multiple

template <int BM, int BN, int WM, int WN, bool LN>
__device__ __forceinline__ void gemm_epilogue_rope72_lds(const GemmParams& p,
                                                         f32x16 (&acc)[GemmShape<BM, BN, WM, WN>::NB][GemmShape<BM, BN, WM, WN>::MB],
                                                         int m0, int n0, int wm, int wn, int lane, int tid, bf16* smem,
                                                         const uint32_t* ltab, const f32x2* lcd) {
  using S = GemmShape<BM, BN, WM, WN>;
  static_assert(BN == 4 * 72 && BM % 8 == 0, "four 72-dim heads per tile");
  const int l32 = lane & 31, hh = lane >> 5;
  LnRows<S::MB> L;
  if constexpr (LN) L = ln_rows<S::MB>(lcd + BN, wm * S::TM + l32);
#pragma unroll
  for (int a = 0; a < S::NB; ++a)
#pragma unroll
    for (int b = 0; b < S::MB; ++b)
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const int r = wm * S::TM + b * 32 + l32;
        const int c = wn * S::TN + a * 32 + 8 * g + 4 * hh;
        float f[4] = {acc[a][b][4 * g], acc[a][b][4 * g + 1], acc[a][b][4 * g + 2], acc[a][b][4 * g + 3]};
        if constexpr (LN) ln_fold_group(lcd, L.r[b], L.nm[b], c, f);
        *reinterpret_cast<u32x2*>(smem + r * kR72 + c) = u32x2{pack_bf16x2(f[0], f[1]), pack_bf16x2(f[2], f[3])};
      }
  __syncthreads();
  const int which = n0 / p.D;                    // tiles never straddle q | k | v (D % 288 == 0)
  const int head0 = (n0 % p.D) / 72;
  if (which < 2) {
    bf16* dst = which == 0 ? p.q : p.k;
    constexpr int ITEMS = BM * 4 * 9;            // (token, head, group of 4 rotary pairs)
    for (int it = tid; it < ITEMS; it += S::THREADS) {
      const int r = it / 36, rem = it % 36, h = rem / 9, d = (rem % 9) * 4;
      const int m = m0 + r;
      if (m >= p.Np) continue;
      const int n = n0 + h * 72 + d;
      const bf16* src = smem + r * kR72 + h * 72 + d;
      const u32x2 lr = *reinterpret_cast<const u32x2*>(src);
      const u32x2 hr = *reinterpret_cast<const u32x2*>(src + 36);
      const float lo[4] = {bf16_lo(lr.x), bf16_hi(lr.x), bf16_lo(lr.y), bf16_hi(lr.y)};
      const float hi[4] = {bf16_lo(hr.x), bf16_hi(hr.x), bf16_lo(hr.y), bf16_hi(hr.y)};
      const f32x4 blo = *reinterpret_cast<const f32x4*>(p.bias + n);
      const f32x4 bhi = *reinterpret_cast<const f32x4*>(p.bias + n + 36);
      f32x4 c01, c23;
      if (ltab) {
        int ph, pw;
        token_pos(p, m, ph, pw);
        rope_cs_table(ltab, 18, ph, pw, d, c01, c23);
      } else {
        rope_cs_global(p, m, d, c01, c23);
      }
      u32x2 o1, o2;
      rope_values(p, which, m, d, blo, bhi, lo, hi, c01, c23, o1, o2);
      bf16* row = dst + ((int64_t)(head0 + h) * p.Np + m) * 88;
      *reinterpret_cast<u32x2*>(row + d) = o1;
      *reinterpret_cast<u32x2*>(row + 36 + d) = o2;
    }
    for (int it = tid; it < BM * 8; it += S::THREADS) {     // dims 72..87: two 16-byte zero runs per row
      const int r = it / 8, h = (it / 2) % 4, half = it % 2;
      const int m = m0 + r;
      if (m < p.Np)
        *reinterpret_cast<u32x4*>(dst + ((int64_t)(head0 + h) * p.Np + m) * 88 + 72 + 8 * half) = u32x4{0u, 0u, 0u, 0u};
    }
  } else {
    constexpr int PCH = BM / 8;                  // 8-position chunks of the tile's V^T rows
    constexpr int ITEMS = 4 * 36 * PCH;          // (head, dim pair, position chunk)
    for (int it = tid; it < ITEMS; it += S::THREADS) {
      const int pc = it % PCH, rest = it / PCH, dp = rest % 36, h = rest / 36;
      const int d = 2 * dp, P = m0 + pc * 8;
      if (P >= p.Np) continue;
      const int n = n0 + h * 72 + d;
      const float b0 = p.bias[n], b1 = p.bias[n + 1];
      float v0[8], v1[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const int m = vt_pos(P + e);             // the token stored at position P + e
        const uint32_t w = *reinterpret_cast<const uint32_t*>(smem + (m - m0) * kR72 + h * 72 + d);
        const bool live = m < p.M;
        v0[e] = live ? bf16_lo(w) + b0 : 0.f;
        v1[e] = live ? bf16_hi(w) + b1 : 0.f;
      }
      bf16* row = p.vt + ((int64_t)(head0 + h) * 72 + d) * p.Np + P;
      *reinterpret_cast<u32x4*>(row) = u32x4{pack_bf16x2(v0[0], v0[1]), pack_bf16x2(v0[2], v0[3]),
                                             pack_bf16x2(v0[4], v0[5]), pack_bf16x2(v0[6], v0[7])};
      *reinterpret_cast<u32x4*>(row + p.Np) = u32x4{pack_bf16x2(v1[0], v1[1]), pack_bf16x2(v1[2], v1[3]),
                                                    pack_bf16x2(v1[4], v1[5]), pack_bf16x2(v1[6], v1[7])};
    }
  }
}

// Tile t -> (row tile, column tile). Tiles are ordered in panels of group_n column tiles, row tile
// by row tile within a panel, so the tiles that one XCD runs in one round (a contiguous range, see
// xcd_remap) form a block of about (cus/8)/group_n row tiles by group_n column tiles, and the
// operand bytes that XCD's L2 fetches per round are ~rows*|x tile| + cols*|w tile| instead of the
// whole weight matrix (row-major order puts all column tiles of 2 row tiles in one round).
__device__ __forceinline__ void tile_coords(int tile, int tiles_m, int tiles_n, int group_n, int& tm, int& tn) {
  const int panel = tile / (tiles_m * group_n);
  const int width = min(group_n, tiles_n - panel * group_n);
  const int r = tile - panel * tiles_m * group_n;
  tm = r / width;
  tn = panel * group_n + r % width;
}

// Dynamic LDS of the GEMM. Elements [0, E): the operand ring (`stages` stages) or the epilogue
// staging, whichever is larger. Above it: for a folded LayerNorm (LN kernels) the tile's BN columns'
// (c, d) then its BM rows' (rstd, -mean * rstd), 8 bytes each; then the rotary epilogues'
// per-position table or the pos-embed epilogue's taps.
template <int BM, int BN, int WM, int WN, int EPI>
__host__ __device__ constexpr int gemm_lds_elems_n(int stages) {
  return (stages * GemmShape<BM, BN, WM, WN>::LDS_ELEMS > (EPI == kEpiQkvRope72 ? BM * kR72 : BM * BN))
             ? stages * GemmShape<BM, BN, WM, WN>::LDS_ELEMS
             : (EPI == kEpiQkvRope72 ? BM * kR72 : BM * BN);
}
template <int BM, int BN, int WM, int WN, int EPI, bool LN>
__host__ __device__ constexpr int gemm_lds_bytes_n(int stages) {
  return (((gemm_lds_elems_n<BM, BN, WM, WN, EPI>(stages) + 7) / 8 * 8) + (LN ? (BN + BM) * 4 : 0)) * 2 +
         (EPI == kEpiQkvRope || EPI == kEpiQkvRope72 ? rope_table_lds_bytes(EPI == kEpiQkvRope ? 64 : 72, LN) : 0) +
         (EPI == kEpiBiasPosEmbed ? BM * 4 * 8 : 0);
}
// Operand-ring stages: three (the DMA runs two k-steps ahead, which hides the latency of operands
// that come cold from HBM behind tiles whose k-step is short) where that fits the 160 KB of LDS;
// else two.
template <int BM, int BN, int WM, int WN, int EPI, bool LN>
__host__ __device__ constexpr int gemm_stages() {
  return gemm_lds_bytes_n<BM, BN, WM, WN, EPI, LN>(3) <= 163840 ? 3 : 2;
}
template <int BM, int BN, int WM, int WN, int EPI, bool LN>
__host__ __device__ constexpr int ln_cd_offset() {
  return (gemm_lds_elems_n<BM, BN, WM, WN, EPI>(gemm_stages<BM, BN, WM, WN, EPI, LN>()) + 7) / 8 * 8;
}
template <int BM, int BN, int WM, int WN, int EPI, bool LN>
__host__ __device__ constexpr int rope_tab_offset() {
  return ln_cd_offset<BM, BN, WM, WN, EPI, LN>() + (LN ? (BN + BM) * 4 : 0);
}

// Waits until at most N of this wave's vector memory operations are outstanding (they complete in
// issue order).
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  static_assert(N >= 0 && N <= 63, "vmcnt range");
  asm volatile("s_waitcnt vmcnt(%0)" :: "I"(N) : "memory");
}
// The same for a wave-uniform count n <= MAX (a scalar branch to the matching immediate).
template <int MAX>
__device__ __forceinline__ void wait_vmcnt_upto(int n) {
  if constexpr (MAX > 0) {
    if (n < MAX) {
      wait_vmcnt_upto<MAX - 1>(n);
      return;
    }
  }
  wait_vmcnt<MAX>();
}

template <int BM, int BN, int WM, int WN, int EPI, bool LN>
__global__ __launch_bounds__(64 * WM * WN, 1) void gemm_bf16_kernel(GemmParams p) {
  using S = GemmShape<BM, BN, WM, WN>;
  extern __shared__ __attribute__((aligned(16))) bf16 smem[];   // [NS][BM+BN][64]
  constexpr int NS = gemm_stages<BM, BN, WM, WN, EPI, LN>();

  // Work assignment: workgroups [0, full_tiles) each own a whole tile (XCD-remapped); the rest
  // own 1/split of the K range of one of the remaining "tail" tiles and write fp32 partials.
  const int tiles_n = (p.N + BN - 1) / BN;
  const int KT = p.K / kBK;
  int tile, kt0 = 0, kt1 = KT, unit = -1;
  if ((int)blockIdx.x < p.full_tiles) {
    tile = xcd_remap(blockIdx.x, p.full_tiles);
  } else {
    unit = blockIdx.x - p.full_tiles;
    tile = p.full_tiles + unit / p.split;
    const int s = unit % p.split;
    kt0 = s * KT / p.split;
    kt1 = (s + 1) * KT / p.split;
  }
  int tm, tn;
  tile_coords(tile, ((p.row1 ? p.row1 : max(p.M, p.Np)) - p.row0 + BM - 1) / BM, tiles_n, p.group_n, tm, tn);
  const int m0 = p.row0 + tm * BM, n0 = tn * BN;

  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wave % WM, wn = wave / WM;
  const int l32 = lane & 31, hh = lane >> 5;


  // Global -> LDS by DMA (buffer_load_dwordx4 ... lds): one wave instruction fills 1 KB = 8 rows
  // of 128 bytes; lane j lands in row R0 + j/8 at physical chunk j%8, so it fetches the logical
  // chunk that the read-side swizzle maps there. Rows past M (or N) lie past the resource's range
  // and arrive as zeros. Lane part of the source offset: one VGPR; row-group and K parts: the
  // uniform soffset. Issued as inline asm: completion is awaited explicitly before the barrier
  // that publishes a stage, so the compiler adds no waits between unrelated LDS reads.
  const int r8 = lane >> 3;
  const int lrow = wave * 8 + r8;                           // row within the 64-row pass
  const int lch = (lane & 7) ^ ((lrow >> 1) & 7);           // logical chunk for this lane
  const uint32_t xv = (uint32_t)(((int64_t)(m0 + lrow) * p.lda + lch * 8) * 2);
  const uint32_t wv = (uint32_t)(((int64_t)(n0 + lrow) * p.K + lch * 8) * 2);
  const u32x4 rxw = rsrc_words(p.x, (uint32_t)((int64_t)p.M * p.lda * 2));
  const u32x4 rww = rsrc_words(p.w, (uint32_t)((int64_t)p.N * p.K * 2));
  const uint32_t lds_base = lds_addr_of(smem);
  // DMA instructions this wave issues per stage (the last pass of an operand may skip it).
  const int dma_per_stage = (BM % S::ROWS_PER_PASS == 0 || (S::XPT - 1) * S::ROWS_PER_PASS + wave * 8 < BM ? S::XPT : S::XPT - 1) +
                            (BN % S::ROWS_PER_PASS == 0 || (S::WPT - 1) * S::ROWS_PER_PASS + wave * 8 < BN ? S::WPT : S::WPT - 1);
  // Wait for every stage but the newest one (its dma_per_stage operations may stay in flight).
  auto wait_all_but_newest = [&]() {
    if constexpr (BM % S::ROWS_PER_PASS == 0 && BN % S::ROWS_PER_PASS == 0)
      wait_vmcnt<S::XPT + S::WPT>();
    else
      wait_vmcnt_upto<S::XPT + S::WPT>(dma_per_stage);
  };
  auto dma_stage = [&](int k0, int stage) {
    const uint32_t xa = lds_base + stage * S::LDS_ELEMS * 2, wa = xa + BM * kBK * 2;
#pragma unroll
    for (int i = 0; i < S::XPT; ++i)
      if (BM % S::ROWS_PER_PASS == 0 || i * S::ROWS_PER_PASS + wave * 8 < BM)   // wave-uniform
        dma16(rxw, xv, (uint32_t)((i * S::ROWS_PER_PASS * p.lda + k0) * 2), xa + (i * S::ROWS_PER_PASS + wave * 8) * kBK * 2);
#pragma unroll
    for (int i = 0; i < S::WPT; ++i)
      if (BN % S::ROWS_PER_PASS == 0 || i * S::ROWS_PER_PASS + wave * 8 < BN)
        dma16(rww, wv, (uint32_t)((i * S::ROWS_PER_PASS * p.K + k0) * 2), wa + (i * S::ROWS_PER_PASS + wave * 8) * kBK * 2);
  };

  // The first k-step's operands (and with three stages the second's) are on their way while the
  // prologue below copies its tables.
  dma_stage(kt0 * kBK, 0);
  if constexpr (NS == 3) {
    if (kt0 + 1 < kt1) dma_stage((kt0 + 1) * kBK, 1);
  }

  // The qkv rotary epilogues' per-position (cos, sin) table, copied once into LDS above the
  // operand ring / staging area (its first barrier below publishes it).
  const uint32_t* ltab = nullptr;
  if constexpr (EPI == kEpiQkvRope || EPI == kEpiQkvRope72) {
    if (p.rtab && unit < 0) {
      uint32_t* t = reinterpret_cast<uint32_t*>(smem + rope_tab_offset<BM, BN, WM, WN, EPI, LN>());
      const int words = p.rtab_pos * (p.cs_half / 2);
      for (int i = tid; i < words; i += S::THREADS) t[i] = p.rtab[i];
      ltab = t;
    }
  }

  // The folded LayerNorm's (c, d) of the tile's columns and (rstd, -mean * rstd) of its rows, copied
  // once into LDS (published by the first barrier below); read by the epilogue, and by the tail
  // units, which write their partials already folded (the reductions then only sum).
  const f32x2* lcd = nullptr;
  if constexpr (LN) {
    {
      f32x2* t = reinterpret_cast<f32x2*>(smem + ln_cd_offset<BM, BN, WM, WN, EPI, LN>());
      for (int i = tid; i < BN + BM; i += S::THREADS) {
        if (i < BN) {
          t[i] = n0 + i < p.N ? p.ln_cd[n0 + i] : f32x2{0.f, 0.f};
        } else {
          const f32x2 st = ln_row(p, m0 + i - BN);
          t[i] = f32x2{st.y, -st.x * st.y};
        }
      }
      lcd = t;
    }
  }

  // kEpiBiasPosEmbed: the tile's rows' 4 bilinear taps (index, weight bits) copied once into LDS above
  // the ring / staging area (published by the first barrier below, read by the epilogue).
  const int2* ltaps = nullptr;
  if constexpr (EPI == kEpiBiasPosEmbed) {
    int2* t = reinterpret_cast<int2*>(smem + rope_tab_offset<BM, BN, WM, WN, EPI, LN>());
    for (int i = tid; i < BM * 4; i += S::THREADS) {
      const int m = m0 + (i >> 2), j = i & 3;
      t[i] = m < p.M ? int2{p.pe_idx[(int64_t)j * p.M + m], __float_as_int(p.pe_w[(int64_t)j * p.M + m])}
                     : int2{0, 0};
    }
    ltaps = t;
  }

  f32x16 acc[S::NB][S::MB];
#pragma unroll
  for (int a = 0; a < S::NB; ++a)
#pragma unroll
    for (int b = 0; b < S::MB; ++b) acc[a][b] = f32x16{};

  // Fragments are double-buffered across k-steps: k-step ks+1 is read from LDS while ks's MFMAs
  // run; sched_group_barrier pins the interleave (MFMA, read, MFMA, read, ...), and the next
  // tile's global loads / LDS stores are threaded between the MFMAs of the first / last k-step.
  constexpr int NFR = S::NB + S::MB;
  bf16x8 fr[2][NFR];
  auto read_frags = [&](const bf16* xs, int ks, int slot) {
    const bf16* ws = xs + BM * kBK;
    const int ch = ks * 2 + hh;
#pragma unroll
    for (int a = 0; a < S::NB; ++a)
      fr[slot][a] = *reinterpret_cast<const bf16x8*>(ws + lds_off(wn * S::TN + a * 32 + l32, ch));
#pragma unroll
    for (int b = 0; b < S::MB; ++b)
      fr[slot][S::NB + b] = *reinterpret_cast<const bf16x8*>(xs + lds_off(wm * S::TM + b * 32 + l32, ch));
  };
  auto mfmas = [&](int slot) {
#pragma unroll
    for (int a = 0; a < S::NB; ++a)
#pragma unroll
      for (int b = 0; b < S::MB; ++b)
        acc[a][b] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(fr[slot][a], fr[slot][S::NB + b], acc[a][b], 0, 0, 0);
  };
  constexpr int NMF = S::NB * S::MB;

  // Stage s of the ring holds k-step kt0 + s (mod NS); a stage is refilled one barrier after its
  // last read. The wait before each barrier lets only the newest stage's DMA stay in flight.
  if (NS == 3 && kt0 + 1 < kt1) wait_all_but_newest(); else wait_dma();
  __syncthreads();
  read_frags(smem, 0, 0);

  int cur = 0;
  for (int kt = kt0; kt < kt1; ++kt) {
    const bf16* xs = smem + cur * S::LDS_ELEMS;
    const bool more = kt + 1 < kt1;
    const int nxt = NS == 3 ? (cur == 2 ? 0 : cur + 1) : (cur ^ 1);
    if constexpr (NS == 3) {
      if (kt + 2 < kt1) dma_stage((kt + 2) * kBK, cur == 0 ? 2 : cur - 1);
    } else {
      if (more) dma_stage((kt + 1) * kBK, nxt);
    }
#pragma unroll
    for (int ks = 0; ks < kBK / 16; ++ks) {
      if (ks + 1 < kBK / 16) read_frags(xs, ks + 1, (ks + 1) & 1);
      mfmas(ks & 1);
      if (ks + 1 < kBK / 16) {
#pragma unroll
        for (int i = 0; i < NMF; ++i) {
          __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
          if (i < NFR) __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
        }
      }
    }
    if (NS == 3 && kt + 2 < kt1) wait_all_but_newest(); else wait_dma();
    __syncthreads();
    if (more) read_frags(smem + nxt * S::LDS_ELEMS, 0, 0);
    cur = nxt;
  }

  if (unit >= 0) {
    // Tail unit: store the fp32 partial row-major within the tile, part[unit][BM][BN]. With a
    // folded LayerNorm the partial is folded here: rstd * acc, plus -mean * rstd * c + d in the
    // first K part only, so the parts sum to the folded value.
    float* dst = p.part + (size_t)unit * BM * BN;
    const bool first = unit % p.split == 0;
#pragma unroll
    for (int a = 0; a < S::NB; ++a)
#pragma unroll
      for (int b = 0; b < S::MB; ++b)
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          const int mm = wm * S::TM + b * 32 + l32, nn = wn * S::TN + a * 32 + 8 * g + 4 * hh;
          float v[4] = {acc[a][b][4 * g], acc[a][b][4 * g + 1], acc[a][b][4 * g + 2], acc[a][b][4 * g + 3]};
          if constexpr (LN) {
            const f32x2 rs = lcd[BN + mm];
            const f32x4 cd01 = *reinterpret_cast<const f32x4*>(lcd + nn);
            const f32x4 cd23 = *reinterpret_cast<const f32x4*>(lcd + nn + 2);
            const float nm = first ? rs.y : 0.f;
            const f32x4 z = {0.f, 0.f, 0.f, 0.f};
            ln_fold_cd(first ? cd01 : z, first ? cd23 : z, rs.x, nm, v);
          }
          *reinterpret_cast<f32x4*>(dst + (size_t)mm * BN + nn) = f32x4{v[0], v[1], v[2], v[3]};
        }
    return;
  }
  if constexpr (EPI == kEpiQkvRope) {
    __syncthreads();                    // every wave is done with the last stage
    gemm_epilogue_rope_lds<BM, BN, WM, WN, LN>(p, acc, m0, n0, wm, wn, lane, wave, smem, ltab, lcd);
  } else if constexpr (EPI == kEpiQkvRope72) {
    gemm_epilogue_rope72_lds<BM, BN, WM, WN, LN>(p, acc, m0, n0, wm, wn, lane, tid, smem, ltab, lcd);
  } else {
    gemm_epilogue_lds<BM, BN, WM, WN, EPI, LN>(p, acc, m0, n0, wm, wn, lane, tid, smem, lcd, ltaps);
  }
}

// Sums the split-K partials of the tail tiles and applies the epilogue, one thread per 4-feature
// quad (per quad pair for the rotary epilogue): fully parallel and coalesced over the partials.
template <int BM, int BN, int EPI>
__global__ __launch_bounds__(256) void gemm_splitk_reduce_kernel(GemmParams p, int tail) {
  constexpr int QPR = (EPI == kEpiQkvRope) ? BN / 8 : BN / 4;   // work items per tile row
  const int64_t per_tile = (int64_t)BM * QPR;
  const int64_t idx = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (idx >= (int64_t)tail * per_tile) return;
  const int t = (int)(idx / per_tile);
  const int rem = (int)(idx % per_tile);
  const int mm = rem / QPR, q = rem % QPR;
  const int nn = (EPI == kEpiQkvRope) ? (q / 8) * 64 + (q % 8) * 4 : q * 4;
  const int tiles_n = (p.N + BN - 1) / BN;
  const int tile = p.full_tiles + t;
  int tm, tn;
  tile_coords(tile, (max(p.M, p.Np) + BM - 1) / BM, tiles_n, p.group_n, tm, tn);
  const int m = tm * BM + mm, n = tn * BN + nn;
  float lo[4] = {0.f, 0.f, 0.f, 0.f}, hi[4] = {0.f, 0.f, 0.f, 0.f};
  for (int s = 0; s < p.split; ++s) {
    const float* src = p.part + ((size_t)(t * p.split + s) * BM + mm) * BN + nn;
    const f32x4 a = *reinterpret_cast<const f32x4*>(src);
#pragma unroll
    for (int e = 0; e < 4; ++e) lo[e] += a[e];
    if constexpr (EPI == kEpiQkvRope) {
      const f32x4 b = *reinterpret_cast<const f32x4*>(src + 32);
#pragma unroll
      for (int e = 0; e < 4; ++e) hi[e] += b[e];
    }
  }
  // (a folded LayerNorm is already in the partials: the tail units fold before storing)
  if constexpr (EPI == kEpiQkvRope) {
    epi_rope_pair(p, m, n, lo, hi);
  } else if constexpr (EPI == kEpiBiasResidual) {
    if (!p.rs_part) {
      epi_store_quad<EPI>(p, m, n, lo);
      return;
    }
    // With the row partials: the 32 lanes of each half wave hold the 32 quads of one 128-column
    // group of one row (a tile row is BN / 4 = 32 or 64 consecutive items; N % 128 == 0), so the
    // group's (sum, sum of squared deviations) of the bf16 outputs reduce across the half wave.
    // Rows past M and groups past N skip as a whole half wave.
    if (m >= p.M || n >= p.N) return;
    const f32x4 bv = *reinterpret_cast<const f32x4*>(p.bias + n);
    const u32x2 r = *reinterpret_cast<const u32x2*>(p.res + (int64_t)m * p.ldr + n);
    float v[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) v[e] = epi_value<EPI>(lo[e], bv[e]);
    v[0] += bf16_lo(r.x); v[1] += bf16_hi(r.x); v[2] += bf16_lo(r.y); v[3] += bf16_hi(r.y);
    const u32x2 o = {pack_bf16x2(v[0], v[1]), pack_bf16x2(v[2], v[3])};
    *reinterpret_cast<u32x2*>(p.y + (int64_t)m * p.ldc + n) = o;
    const float y[4] = {bf16_lo(o.x), bf16_hi(o.x), bf16_lo(o.y), bf16_hi(o.y)};
    float sum = (y[0] + y[1]) + (y[2] + y[3]);
#pragma unroll
    for (int off = 1; off < 32; off <<= 1) sum += __shfl_xor(sum, off);
    const float mean = sum * (1.0f / 128.0f);
    float q2 = 0.f;
#pragma unroll
    for (int e = 0; e < 4; ++e) q2 = fmaf(y[e] - mean, y[e] - mean, q2);
#pragma unroll
    for (int off = 1; off < 32; off <<= 1) q2 += __shfl_xor(q2, off);
    if ((threadIdx.x & 31) == 0) p.rs_part[(int64_t)m * (p.N / 128) + n / 128] = f32x2{sum, q2};
  } else {
    epi_store_quad<EPI>(p, m, n, lo);
  }
}

// The split-K reduction of the head_dim-72 rotary qkv GEMM (256 x 288 tiles, 4 heads of one of q, k,
// v each): the tail tiles' fp32 partials (a folded LayerNorm already applied) summed over their K
// parts, then the rope72 epilogue's arithmetic (bias, the reference's roundings, rotary, q
// pre-scale). q / k tiles:
// one thread per (token, head, 4 rotary pairs), dims d..d+3 and d+36..d+39, the group d = 32 also
// zeroing dims 72..87 of the 88-wide rows; v tiles: one thread per (head, dim pair, 8 key
// positions), 16-byte runs of V^T at the vt_pos positions. Tokens in [M, Np) get zeros.
template <int BM, int BN>
__global__ __launch_bounds__(256) void gemm_splitk_reduce_rope72_kernel(GemmParams p, int tail) {
  static_assert(BN == 4 * 72 && BM % 8 == 0, "four 72-dim heads per tile");
  constexpr int QK_ITEMS = BM * 4 * 9, V_ITEMS = 4 * 36 * (BM / 8);
  const int64_t idx = (int64_t)blockIdx.x * 256 + threadIdx.x;
  const int t = (int)(idx / QK_ITEMS);
  const int it = (int)(idx % QK_ITEMS);
  if (t >= tail) return;
  int tm, tn;
  tile_coords(p.full_tiles + t, (max(p.M, p.Np) + BM - 1) / BM, (p.N + BN - 1) / BN, p.group_n, tm, tn);
  const int m0 = tm * BM, n0 = tn * BN;
  const int which = n0 / p.D, head0 = (n0 % p.D) / 72;
  const float* part = p.part + (size_t)t * p.split * BM * BN;
  auto sum4 = [&](int r, int c, float (&a)[4]) {
#pragma unroll
    for (int e = 0; e < 4; ++e) a[e] = 0.f;
    for (int s = 0; s < p.split; ++s) {
      const f32x4 v = *reinterpret_cast<const f32x4*>(part + ((size_t)s * BM + r) * BN + c);
#pragma unroll
      for (int e = 0; e < 4; ++e) a[e] += v[e];
    }
  };
  // (a folded LayerNorm is already in the partials: the tail units fold before storing)
  if (which < 2) {
    const int r = it / 36, rem = it % 36, h = rem / 9, d = (rem % 9) * 4;
    const int m = m0 + r;
    if (m >= p.Np) return;
    const int n = n0 + h * 72 + d;
    float lo[4], hi[4];
    sum4(r, h * 72 + d, lo);
    sum4(r, h * 72 + d + 36, hi);
    // (rope_values rounds the sums to bf16 before the bias, as the GEMM's staging does)
    const f32x4 blo = *reinterpret_cast<const f32x4*>(p.bias + n);
    const f32x4 bhi = *reinterpret_cast<const f32x4*>(p.bias + n + 36);
    f32x4 c01, c23;
    rope_cs_global(p, m, d, c01, c23);
    u32x2 o1, o2;
    rope_values(p, which, m, d, blo, bhi, lo, hi, c01, c23, o1, o2);
    bf16* row = (which == 0 ? p.q : p.k) + ((int64_t)(head0 + h) * p.Np + m) * 88;
    *reinterpret_cast<u32x2*>(row + d) = o1;
    *reinterpret_cast<u32x2*>(row + 36 + d) = o2;
    if (d == 32) {
      *reinterpret_cast<u32x4*>(row + 72) = u32x4{0u, 0u, 0u, 0u};
      *reinterpret_cast<u32x4*>(row + 80) = u32x4{0u, 0u, 0u, 0u};
    }
    return;
  }
  if (it >= V_ITEMS) return;
  // (dim pairs fastest: the lanes of a wave read one partial row's consecutive columns)
  const int dp = it % 36, rest = it / 36, h = rest % 4, pc = rest / 4;
  const int d = 2 * dp, P = m0 + pc * 8;
  if (P >= p.Np) return;
  const int n = n0 + h * 72 + d;
  const float b0 = p.bias[n], b1 = p.bias[n + 1];
  float v0[8], v1[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    const int m = vt_pos(P + e);               // the token stored at position P + e
    float a0 = 0.f, a1 = 0.f;
    for (int s = 0; s < p.split; ++s) {
      const f32x2 v = *reinterpret_cast<const f32x2*>(part + ((size_t)s * BM + (m - m0)) * BN + h * 72 + d);
      a0 += v.x;
      a1 += v.y;
    }
    if (m < p.M) {
      round_bf16_pair(a0, a1);
      v0[e] = a0 + b0;
      v1[e] = a1 + b1;
    } else {
      v0[e] = 0.f;
      v1[e] = 0.f;
    }
  }
  bf16* row = p.vt + ((int64_t)(head0 + h) * 72 + d) * p.Np + P;
  *reinterpret_cast<u32x4*>(row) = u32x4{pack_bf16x2(v0[0], v0[1]), pack_bf16x2(v0[2], v0[3]),
                                         pack_bf16x2(v0[4], v0[5]), pack_bf16x2(v0[6], v0[7])};
  *reinterpret_cast<u32x4*>(row + p.Np) = u32x4{pack_bf16x2(v1[0], v1[1]), pack_bf16x2(v1[2], v1[3]),
                                                pack_bf16x2(v1[4], v1[5]), pack_bf16x2(v1[6], v1[7])};
}

// Compute units of the current device. A write-once per-device cache: every thread that fills
// an entry stores the same value (relaxed atomics, no other shared state).
int gemm_device_cus() {
  static std::atomic<int> cus[64];
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  int n = cus[dev].load(std::memory_order_relaxed);
  if (n == 0) {
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0) n = 256;
    cus[dev].store(n, std::memory_order_relaxed);
  }
  return n;
}

// Work plan for BM x BN tiles, one workgroup per CU (every tile shape takes 96-136 KB of LDS).
// Cost model, in microseconds: a tile costs BM*BN*K MACs at a per-CU rate `tile_rate` measured
// with every CU busy; whole rounds of tiles run as is; the last partial round either runs as is
// or, with a partials workspace, is split along K so its units fill one round (1/split of a tile)
// plus the split-K reduction, priced at its fp32 partial traffic (written once, read once; the
// partials mostly stay in L2 / MALL). The chip is power-limited: with a fraction f of the CUs
// busy the clock rises until it caps, so a round with f below kRoundFloor takes kRoundFloor of
// a full round's time, not f of it (measured: 128 tiles of 288x256x4096 on 256 CUs run at 2.6x
// the per-CU rate of a full round).
struct GemmPlan { int full, split, tail; double cost_us; };

constexpr double kPartialBytesPerUs = 16.0e6;
constexpr double kReduceLaunchUs = 4.0;
constexpr double kRoundFloor = 0.65;

static double round_fraction(int units, int cus) { return std::max((double)units / cus, kRoundFloor); }

template <int BM, int BN>
static GemmPlan plan_gemm(const GemmParams& p, int cus, double macs_per_us_per_cu, int split_mode) {
  // (the rotary epilogue also zero-fills [M, Np))
  const int rows = (p.row1 ? p.row1 : std::max(p.M, p.Np)) - p.row0;
  const int tiles = ((rows + BM - 1) / BM) * ((p.N + BN - 1) / BN);
  const int KT = p.K / kBK;
  const double tile_us = (double)BM * BN * p.K / macs_per_us_per_cu;
  const int tail = tiles % cus;
  GemmPlan g{tiles, 1, 0, (tiles / cus) * tile_us + (tail ? round_fraction(tail, cus) * tile_us : 0.0)};
  if (tail == 0 || !p.part || split_mode < 0 || p.row0 || p.row1) return g;
  int split = std::min(std::min(8, KT), cus / tail);
  while (split >= 2 && (int64_t)tail * split * BM * BN > p.part_elems) --split;   // what the workspace holds
  if (split < 2) return g;
  const double part_bytes = 2.0 * tail * split * BM * BN * sizeof(float);
  const double cost = (tiles / cus) * tile_us + round_fraction(tail * split, cus) * tile_us / split +
                      part_bytes / kPartialBytesPerUs + kReduceLaunchUs;
  if (cost >= g.cost_us && split_mode == 0) return g;
  g.full = tiles - tail;
  g.tail = tail;
  g.split = split;
  g.cost_us = cost;
  return g;
}

// Tile-plan override of the calling thread (qvl_set_gemm_plan): tile 0 = the cost model's
// choice, 1..4 = 288x256 | 256x256 | 256x128 | 288x128, 5 = the row split (whole rounds of 288x256,
// the rest 256x128), 6 = 128x128, 7 = 64x192 (the head_dim-64 rotary qkv GEMM only), 8 = 64x128;
// split_mode -1 forbids, 1 forces, 0 lets the cost model decide the tail split;
// group_n 0 = the default panel width. Thread-local, so a test pinning a plan on one thread does
// not change another thread's launches.
struct ForcedPlan { int tile = 0, split_mode = 0, group_n = 0; };
static thread_local ForcedPlan t_plan;

// Column tiles per panel of the tile order.
static int gemm_group_n(int tiles_n) {
  const int g = t_plan.group_n > 0 ? t_plan.group_n : 4;
  return std::max(1, std::min(g, tiles_n));
}

template <int BM, int BN, int WM, int WN, int EPI, bool LN>
static int launch_gemm(GemmParams p, const GemmPlan& g, hipStream_t stream) {
  using S = GemmShape<BM, BN, WM, WN>;
  constexpr bool kRope = EPI == kEpiQkvRope || EPI == kEpiQkvRope72;
  // rotary epilogues: room for the largest position table (rope_table_lds_bytes) after the ring
  // (and the folded LayerNorm's (c, d))
  // (the pos-embed epilogue's tap table takes the same place: BM rows x 4 taps x 8 bytes)
  constexpr size_t pe_taps = EPI == kEpiBiasPosEmbed ? (size_t)BM * 4 * 8 : 0;
  constexpr size_t lds_max = (size_t)rope_tab_offset<BM, BN, WM, WN, EPI, LN>() * sizeof(bf16) +
                             (kRope ? rope_table_lds_bytes(EPI == kEpiQkvRope ? 64 : 72, LN) : 0) + pe_taps;
  static_assert(lds_max == (size_t)gemm_lds_bytes_n<BM, BN, WM, WN, EPI, LN>(gemm_stages<BM, BN, WM, WN, EPI, LN>()),
                "LDS layout");
  static_assert(lds_max <= 163840, "LDS budget");
  const size_t lds = p.rtab ? lds_max : (size_t)rope_tab_offset<BM, BN, WM, WN, EPI, LN>() * sizeof(bf16) + pe_taps;
  // once per instantiation (a C++ function-local static: initialised exactly once, thread-safe)
  static const hipError_t attr_rc = hipFuncSetAttribute((const void*)gemm_bf16_kernel<BM, BN, WM, WN, EPI, LN>,
                                                        hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds_max);
  if (attr_rc != hipSuccess) return set_error(QVL_ERR_LAUNCH, "gemm_bf16: cannot reserve %zu bytes of LDS", lds_max);
  p.full_tiles = g.full;
  p.split = g.split;
  p.group_n = gemm_group_n((p.N + BN - 1) / BN);
  const int grid = g.full + g.tail * g.split;
  hipLaunchKernelGGL((gemm_bf16_kernel<BM, BN, WM, WN, EPI, LN>), dim3(grid), dim3(S::THREADS), lds, stream, p);
  int rc = check_launch("gemm_bf16");
  if (rc || g.tail == 0) return rc;
  if constexpr (EPI == kEpiBiasPosEmbed) {
    return set_error(QVL_ERR_INVALID_ARG, "gemm_bf16: the pos-embed epilogue has no split-K tail");
  } else if constexpr (EPI == kEpiQkvRope72) {
    const int64_t items = (int64_t)g.tail * BM * 4 * 9;
    hipLaunchKernelGGL((gemm_splitk_reduce_rope72_kernel<BM, BN>), dim3((unsigned)((items + 255) / 256)), dim3(256), 0,
                       stream, p, g.tail);
    return check_launch("gemm_splitk_reduce_rope72");
  } else {
  const int64_t items = (int64_t)g.tail * BM * ((EPI == kEpiQkvRope) ? BN / 8 : BN / 4);
  hipLaunchKernelGGL((gemm_splitk_reduce_kernel<BM, BN, EPI>), dim3((unsigned)((items + 255) / 256)), dim3(256), 0,
                     stream, p, g.tail);
  return check_launch("gemm_splitk_reduce");
  }
}

// Tile choice by the cost model above. Shapes (per-CU MAC rates measured on the tower's GEMMs):
//   288x256 on 12 waves (three per SIMD, 96x64 each): 64 row tiles cover 18432 tokens, so the
//     N = 1024 / 3072 / 4096 GEMMs fill exactly 1 / 3 / 4 rounds of 256 CUs;
//   256x256 on 8 waves (two per SIMD, 64x128 each): the least LDS traffic per MFMA;
//   256x128 on 8 waves (64x64 each): half the work per tile, for balancing small grids (its
//     three-stage ring keeps it fed on cold weights; with it the 8192-token qkv's 3 rounds of
//     these beat 1.5 rounds of 256x256: 70 against 74 us; the row split below, one round of
//     288x256 and 216 tiles of these, is what that GEMM now runs);
//   288x128 on 12 waves (96x32 each): fills the CUs where 288x256 tiles would cover only half
//     of them (the merger's 4608 x 2048 output is exactly 256 such tiles);
//   128x128 on 4 waves (64x64 each, one per SIMD): small grids, by the rule in dispatch_gemm.
constexpr double kRate288x256 = 1.50e6, kRate256x256 = 1.50e6, kRate256x128 = 1.42e6,
                 kRate288x128 = 1.36e6, kRate128x128 = 1.0e6;   // MACs/us/CU
constexpr int kSmallTileMaxK = 1536;

template <int EPI, bool LN>
static int dispatch_gemm(const GemmParams& p, hipStream_t stream) {
  const int cus = gemm_device_cus();
  ForcedPlan f = t_plan;
  // the split-K reduction computes no pos-embed
  if (EPI == kEpiBiasPosEmbed) f.split_mode = -1;
  const GemmPlan a = plan_gemm<288, 256>(p, cus, kRate288x256, f.split_mode);
  const GemmPlan b = plan_gemm<256, 256>(p, cus, kRate256x256, f.split_mode);
  const GemmPlan c = plan_gemm<256, 128>(p, cus, kRate256x128, f.split_mode);
  const GemmPlan d = plan_gemm<288, 128>(p, cus, kRate288x128, f.split_mode);
  // Row split: the rows that fill whole rounds of 288x256 tiles in one launch, the rest in 256x128
  // tiles in a second launch that fits one round (GemmParams::row0 / row1; no split-K tail). The
  // k order of every output is that of the other plans, so the outputs are the same bits.
  const int rows = std::max(p.M, p.Np), tiles_n_a = (p.N + 255) / 256;
  const int whole_rows = (((rows + 287) / 288) * tiles_n_a / cus) * cus / tiles_n_a * 288;
  GemmParams ra = p, rb = p;
  ra.row1 = whole_rows;
  rb.row0 = whole_rows;
  rb.row1 = rows;
  const bool can_split = whole_rows > 0 && whole_rows < rows && !p.row0 && !p.row1;
  const GemmPlan r_a = plan_gemm<288, 256>(ra, cus, kRate288x256, -1);
  const GemmPlan r_b = plan_gemm<256, 128>(rb, cus, kRate256x128, -1);
  const double r_cost = can_split && r_b.full <= cus ? r_a.cost_us + r_b.cost_us : 1e30;
  int pick = f.tile;
  if (EPI == kEpiQkvRope && pick == 4) pick = 3;     // 64-feature heads need TN % 64 == 0 (288x128: 32)
  if (pick == 5 && !can_split) pick = 1;
  // Small grids, K <= 1536: where one round of 128x128 tiles would cover half to all of the CUs,
  // 64x128 tiles unsplit (4 waves of 32x64); where fewer 128x128 tiles split along K in up to 8
  // parts fill at least 7/8 of the CUs, those (4 waves of 64x64). The larger tiles there leave most
  // CUs idle or need long split-K tails. One 784-token image's forward: fc1 16.1 us on 128x128
  // against 21.3 on 256x128 (64x128: below); proj, 56 tiles in 4 parts, 15.4 against 18.9 us for
  // 288x128 tiles in 8 parts. Cases the rules leave to the cost model were measured slower on
  // 128x128: 1568 rows' proj unsplit (104 tiles) 22.9 against 20.4 us; the mergers' K = 4096 GEMMs
  // at 196 rows 25.2 / 26.8 against 20.3 / 24.2 us.
  // The head_dim-64 rotary qkv GEMM takes 64x192 tiles (6 waves of 32x64, whole heads; tiles may
  // straddle the q | k | v boundary, the epilogue picks the target per head) wherever one round of
  // them fits the CUs: alone on MI355X (1024 x 3072 x 1024 with norm1 folded), 196 / 400 / 576 /
  // 784 / 1024 tokens 14.3 / 14.5 / 14.7 / 15.3 / 15.4 us against 19.8 / 20.2 / 20.2 / 17.0 / 17.5
  // for the plans below; at 1568 tokens and more (two rounds) the plans below stay ahead.
  GemmPlan e{};
  if (pick == 6) e = plan_gemm<128, 128>(p, cus, kRate128x128, f.split_mode);
  if constexpr (EPI == kEpiQkvRope) {
    const int tiles64 = ((rows + 63) / 64) * ((p.N + 191) / 192);
    if (pick == 0 && p.K <= kSmallTileMaxK && tiles64 <= cus && !p.row0 && !p.row1) pick = 7;
  }
  const int tiles128 = ((rows + 127) / 128) * ((p.N + 127) / 128);
  if (pick == 0 && p.K <= kSmallTileMaxK && !p.row0 && !p.row1) {
    if (2 * tiles128 >= cus && tiles128 <= cus) {
      // below a full round of 128x128 tiles, one to two rounds of 64x128 run ahead (alone: fc1 at
      // 784 rows 14.8 against 15.8 us, the 8B fc1 16.3 against 17.2, proj at 2304 rows 16.1 against
      // 20.6; in the forward a 2304-patch image 4.013 -> 3.889 ms); a full round stays on 128x128
      // (fc1 at 1024 rows: two full rounds of 64x128 made the forward 0.9 % slower); the head_dim-64
      // rotary qkv stays on 128x128 (64x128: 24-26 against 17.7 us at 784 tokens)
      if (tiles128 < cus && EPI != kEpiQkvRope) {
        pick = 8;
        e = plan_gemm<64, 128>(p, cus, kRate128x128, -1);
      } else {
        pick = 6;
        e = plan_gemm<128, 128>(p, cus, kRate128x128, -1);
      }
    } else if (f.split_mode >= 0 && 2 * tiles128 < cus) {
      const GemmPlan sp = plan_gemm<128, 128>(p, cus, kRate128x128, 1);
      if (8 * sp.tail * sp.split >= 7 * cus) {
        pick = 6;
        e = sp;
      }
    } else if (EPI == kEpiBiasPosEmbed && ((rows + 63) / 64) * ((p.N + 127) / 128) <= cus) {
      // the patch embed cannot split K: its small grids take 64x128 tiles (4 waves of 32x64) that
      // fit one round (one 784-token image: 104 tiles, 23.5 against 37.9 us for 32 of 256x128)
      pick = 8;
    }
  }
  // Long K (fc2, K = 4096 / 4352) from 512 rows: 128x128 tiles split along K where up to 8 parts fill
  // at least 7/8 of the CUs (one 784-token image's fc2: 23.9 against 25.2 us for 288x128 tiles in 8
  // parts); at the mergers' 196 rows the cost model's plans stay ahead (25.2 / 26.8 against 20.3 /
  // 24.2 us on 128x128).
  if (pick == 0 && p.K > kSmallTileMaxK && rows >= 512 && f.split_mode >= 0 && !p.row0 && !p.row1 &&
      EPI != kEpiBiasPosEmbed && 2 * tiles128 < cus) {
    const GemmPlan sp = plan_gemm<128, 128>(p, cus, kRate128x128, 1);
    if (8 * sp.tail * sp.split >= 7 * cus) {
      pick = 6;
      e = sp;
    }
  }
  // A folded LayerNorm over more than 16 row groups (the deepstack mergers' 4-token rows: 32 or 36)
  // combines each row's partials in the workgroup's prologue; on small grids 64-row tiles split
  // along K spread that over 4x the workgroups (one 784-token image's deepstack fc1, K = 4096:
  // 27.2 against 33.4 us for 256x128 tiles split 8 ways).
  if (pick == 0 && LN && p.ln_part && p.ln_groups > 16 && f.split_mode >= 0 && !p.row0 && !p.row1 &&
      2 * ((rows + 63) / 64) * ((p.N + 127) / 128) <= cus) {
    const GemmPlan sp = plan_gemm<64, 128>(p, cus, kRate128x128, 1);
    if (8 * sp.tail * sp.split >= 7 * cus) {
      pick = 8;
      e = sp;
    }
  }
  if (pick == 0) {
    const double cost[5] = {a.cost_us, b.cost_us, c.cost_us, EPI == kEpiQkvRope ? 1e30 : d.cost_us, r_cost};
    pick = 1;
    for (int i = 1; i < 5; ++i)
      if (cost[i] < cost[pick - 1]) pick = i + 1;
  }
  if (pick == 5) {
    const int rc = launch_gemm<288, 256, 3, 4, EPI, LN>(ra, r_a, stream);
    if (rc) return rc;
    return launch_gemm<256, 128, 4, 2, EPI, LN>(rb, r_b, stream);
  }
  if (pick == 1) return launch_gemm<288, 256, 3, 4, EPI, LN>(p, a, stream);
  if (pick == 6) return launch_gemm<128, 128, 2, 2, EPI, LN>(p, e, stream);
  if constexpr (EPI == kEpiQkvRope) {
    if (pick == 7) return launch_gemm<64, 192, 2, 3, EPI, LN>(p, plan_gemm<64, 192>(p, cus, kRate128x128, -1), stream);
  }
  if (pick == 8)
    return launch_gemm<64, 128, 2, 2, EPI, LN>(p, e.full || e.tail ? e : plan_gemm<64, 128>(p, cus, kRate128x128, f.split_mode),
                                               stream);
  if constexpr (EPI == kEpiQkvRope) {
    if (pick == 3) return launch_gemm<256, 128, 4, 2, EPI, LN>(p, c, stream);
    return launch_gemm<256, 256, 4, 2, EPI, LN>(p, b, stream);
  } else {
    if (pick == 2) return launch_gemm<256, 256, 4, 2, EPI, LN>(p, b, stream);
    if (pick == 3) return launch_gemm<256, 128, 4, 2, EPI, LN>(p, c, stream);
    return launch_gemm<288, 128, 3, 4, EPI, LN>(p, d, stream);
  }
}

int gemm_set_plan(int tile, int split_mode, int group_n) {
  if (tile < 0 || tile > 8 || split_mode < -1 || split_mode > 1 || group_n < 0)
    return set_error(QVL_ERR_INVALID_ARG, "gemm plan: tile=%d split_mode=%d group_n=%d", tile, split_mode, group_n);
  t_plan.tile = tile;
  t_plan.split_mode = split_mode;
  t_plan.group_n = group_n;
  return QVL_OK;
}

// head_dim-72 qkv GEMM: 256 x 288 tiles (4 heads each, 12 waves of 64 x 96). Where those tiles leave
// a last round at most half full and the rows past the whole rounds fit one round of 128 x 288 tiles
// (12 waves of 32 x 96), the rows run in two launches: whole rounds of 256-row tiles, then the rest
// in 128-row tiles, so the last round does half a tile's work per CU (config 4: 336 tiles on 256
// CUs become 252 + 168 half tiles; the outputs are the same bits, as the k order is). The last
// partial round can instead be split along K when a plan forces it
// (gemm_splitk_reduce_rope72_kernel applies the epilogue): at config 4 the split ran its GEMM in 76
// us and the reduction of the 47 MB of fp32 partials in 16 us, against 91-93 us unsplit (MI355X).
// Small grids, where the 128-row launch would fill at most half of the CUs and 64-row tiles fit one
// round, take 64 x 288 tiles (6 waves of 32 x 96) for those rows instead (one 784-token image: 156
// tiles against 84). Plan override (qvl_set_gemm_plan's tile): 1 = one launch of 256 x 288 tiles,
// 2 = the row split wherever there are two row tiles (the 128-row launch alone when no whole round
// exists), 3 = the same with 64-row tiles for the rows past the whole rounds.
constexpr double kRate256x288 = 1.50e6;

template <bool LN>
static int launch_qkv_rope72(const GemmParams& p, hipStream_t stream) {
  const int cus = gemm_device_cus();
  const int rows = std::max(p.M, p.Np), tiles_n = (p.N + 287) / 288;
  const int row_tiles = (rows + 255) / 256, tiles = row_tiles * tiles_n, tail = tiles % cus;
  const int whole_rows = (tiles / cus) * cus / tiles_n * 256;          // rows in whole rounds
  const int half_tiles = (rows - whole_rows + 127) / 128 * tiles_n;    // the rest in 128-row tiles
  const int quarter_tiles = (rows - whole_rows + 63) / 64 * tiles_n;   // or in 64-row tiles
  const bool row_split = t_plan.split_mode != 1 && t_plan.tile != 1 && row_tiles >= 2 &&
                         (t_plan.tile == 2 || t_plan.tile == 3 || (tail && 2 * tail <= cus && half_tiles <= cus));
  const bool quarter = t_plan.tile == 3 || (t_plan.tile == 0 && 2 * half_tiles <= cus && quarter_tiles <= cus);
  if (!row_split) {
    const GemmPlan g = plan_gemm<256, 288>(p, cus, kRate256x288, t_plan.split_mode == 1 ? 1 : -1);
    return launch_gemm<256, 288, 4, 3, kEpiQkvRope72, LN>(p, g, stream);
  }
  GemmParams a = p, b = p;
  a.row0 = 0;
  a.row1 = whole_rows;
  b.row0 = whole_rows;
  b.row1 = rows;
  if (whole_rows > 0) {
    const int rc = launch_gemm<256, 288, 4, 3, kEpiQkvRope72, LN>(a, plan_gemm<256, 288>(a, cus, kRate256x288, -1), stream);
    if (rc) return rc;
  }
  if (quarter)
    return launch_gemm<64, 288, 2, 3, kEpiQkvRope72, LN>(b, plan_gemm<64, 288>(b, cus, kRate256x288, -1), stream);
  return launch_gemm<128, 288, 4, 3, kEpiQkvRope72, LN>(b, plan_gemm<128, 288>(b, cus, kRate256x288, -1), stream);
}

static int dispatch_qkv_rope72(const GemmParams& p, hipStream_t stream) {
  if (p.ln_stats || p.ln_part) return launch_qkv_rope72<true>(p, stream);
  return launch_qkv_rope72<false>(p, stream);
}

// A folded LayerNorm (p.ln_stats or p.ln_part) selects the kernels instantiated with the fold (bias, GELU and
// rotary epilogues: the Dense layers that follow a LayerNorm); the others carry no trace of it.
int gemm_bf16(const GemmParams& p, int epi, hipStream_t stream) {
  const bool ln = p.ln_stats != nullptr || p.ln_part != nullptr;
  if (p.rs_part && ((epi != kEpiBiasResidual && epi != kEpiBiasPosEmbed) || p.N % 128))
    return set_error(QVL_ERR_INVALID_ARG, "gemm_bf16: row statistics need the residual epilogue and N %% 128 == 0");
  if (ln && !p.ln_cd) return set_error(QVL_ERR_INVALID_ARG, "gemm_bf16: folded LayerNorm without (c, d)");
  switch (epi) {
    case kEpiQkvRope72: return dispatch_qkv_rope72(p, stream);
    case kEpiBias: return ln ? dispatch_gemm<kEpiBias, true>(p, stream) : dispatch_gemm<kEpiBias, false>(p, stream);
    case kEpiBiasGelu:
      return ln ? dispatch_gemm<kEpiBiasGelu, true>(p, stream) : dispatch_gemm<kEpiBiasGelu, false>(p, stream);
    case kEpiBiasResidual:
      if (ln) return set_error(QVL_ERR_INVALID_ARG, "gemm_bf16: no folded LayerNorm with the residual epilogue");
      return dispatch_gemm<kEpiBiasResidual, false>(p, stream);
    case kEpiBiasPosEmbed:
      if (ln || !p.pe_table || !p.pe_idx || !p.pe_w || p.N % 8 || p.ldc % 8)
        return set_error(QVL_ERR_INVALID_ARG, "gemm_bf16: pos-embed epilogue operands");
      return dispatch_gemm<kEpiBiasPosEmbed, false>(p, stream);
    case kEpiQkvRope:
      return ln ? dispatch_gemm<kEpiQkvRope, true>(p, stream) : dispatch_gemm<kEpiQkvRope, false>(p, stream);
  }
  return set_error(QVL_ERR_INVALID_ARG, "unknown epilogue %d", epi);
}

}  // namespace qvl
