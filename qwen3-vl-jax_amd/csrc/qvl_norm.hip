// Memory-bound kernels of the vision tower: LayerNorm, learned pos-embed interpolation, the
// rotary (cos, sin) table, the fp32 -> bf16 cast of pixel patches and load-time weight packing.
// Each is HBM-bound; all use 16-byte vector accesses along the contiguous feature axis.
#include <math.h>
#include "qvl_kernels.h"

namespace qvl {

// ---------------------------------------------------------------------------------------------
// LayerNorm (model.py:375-388): one wave per row, row held in registers (CH 16-byte chunks per
// lane), exact two-pass mean / biased variance in fp32, rsqrt(var + eps), affine, bf16 out.
// Each wave walks rows row0, row0 + stride, ... (a grid of ~4 workgroups per CU) with gamma /
// beta held in registers and the next row's loads issued before the current row's reductions:
// 12.7 us for 18432 x 1024 against 15.1 us for one short-lived wave per row (a plain copy of
// the same bytes takes 11.5 us).
// ---------------------------------------------------------------------------------------------
__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) v += __shfl_xor(v, o);
  return v;
}

template <int CH>
__global__ __launch_bounds__(256) void layernorm_bf16_kernel(const bf16* __restrict__ x, int64_t ldx,
                                                             const float* __restrict__ gamma,
                                                             const float* __restrict__ beta,
                                                             bf16* __restrict__ y, int64_t ldy, int rows,
                                                             int cols, float eps) {
  const int lane = threadIdx.x & 63;
  const int stride = gridDim.x * 4;
  const int nch = cols >> 3;
  // gamma / beta: held in registers for rows up to 2048 features, re-read (L1 / L2 hits) above.
  constexpr bool kHold = CH <= 4;
  f32x4 g[kHold ? CH : 1][2], b[kHold ? CH : 1][2];
  if constexpr (kHold) {
#pragma unroll
    for (int i = 0; i < CH; ++i) {
      const int c = lane + 64 * i;
      if (c < nch) {
        g[i][0] = *reinterpret_cast<const f32x4*>(gamma + c * 8);
        g[i][1] = *reinterpret_cast<const f32x4*>(gamma + c * 8 + 4);
        b[i][0] = *reinterpret_cast<const f32x4*>(beta + c * 8);
        b[i][1] = *reinterpret_cast<const f32x4*>(beta + c * 8 + 4);
      }
    }
  }
  const float inv_n = 1.0f / (float)cols;
  auto load_row = [&](int r, u32x4* dst) {
    const bf16* xr = x + (int64_t)r * ldx;
#pragma unroll
    for (int i = 0; i < CH; ++i) {
      const int c = lane + 64 * i;
      dst[i] = (c < nch) ? *reinterpret_cast<const u32x4*>(xr + c * 8) : u32x4{0u, 0u, 0u, 0u};
    }
  };
  int row = blockIdx.x * 4 + (threadIdx.x >> 6);
  u32x4 nxt[CH];
  if (row < rows) load_row(row, nxt);
  for (; row < rows; row += stride) {
    float v[CH][8];
    float s = 0.f;
#pragma unroll
    for (int i = 0; i < CH; ++i) {
      const u32x4 w = nxt[i];
      v[i][0] = bf16_lo(w.x); v[i][1] = bf16_hi(w.x); v[i][2] = bf16_lo(w.y); v[i][3] = bf16_hi(w.y);
      v[i][4] = bf16_lo(w.z); v[i][5] = bf16_hi(w.z); v[i][6] = bf16_lo(w.w); v[i][7] = bf16_hi(w.w);
#pragma unroll
      for (int e = 0; e < 8; ++e) s += v[i][e];      // chunks past the row end hold zeros
    }
    if (row + stride < rows) load_row(row + stride, nxt);
    const float mean = wave_sum(s) * inv_n;
    float q = 0.f;
#pragma unroll
    for (int i = 0; i < CH; ++i) {
      const int c = lane + 64 * i;
      if (c < nch) {
#pragma unroll
        for (int e = 0; e < 8; ++e) { const float d = v[i][e] - mean; q += d * d; }
      }
    }
    const float var = wave_sum(q) * inv_n;
    const float rstd = rsqrtf(var + eps);
    bf16* yr = y + (int64_t)row * ldy;
#pragma unroll
    for (int i = 0; i < CH; ++i) {
      const int c = lane + 64 * i;
      if (c < nch) {
        f32x4 g0, g1, b0, b1;
        if constexpr (kHold) {
          g0 = g[i][0]; g1 = g[i][1]; b0 = b[i][0]; b1 = b[i][1];
        } else {
          g0 = *reinterpret_cast<const f32x4*>(gamma + c * 8);
          g1 = *reinterpret_cast<const f32x4*>(gamma + c * 8 + 4);
          b0 = *reinterpret_cast<const f32x4*>(beta + c * 8);
          b1 = *reinterpret_cast<const f32x4*>(beta + c * 8 + 4);
        }
        float o[8];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          o[e] = (v[i][e] - mean) * rstd * g0[e] + b0[e];
          o[4 + e] = (v[i][4 + e] - mean) * rstd * g1[e] + b1[e];
        }
        u32x4 w = {pack_bf16x2(o[0], o[1]), pack_bf16x2(o[2], o[3]), pack_bf16x2(o[4], o[5]),
                   pack_bf16x2(o[6], o[7])};
        *reinterpret_cast<u32x4*>(yr + c * 8) = w;
      }
    }
  }
}

template <int CH>
static int launch_ln(const bf16* x, int64_t ldx, const float* g, const float* b, bf16* y, int64_t ldy,
                     int rows, int cols, float eps, hipStream_t stream) {
  const int grid = std::min((rows + 3) / 4, 4 * gemm_device_cus());
  hipLaunchKernelGGL(layernorm_bf16_kernel<CH>, dim3(grid), dim3(256), 0, stream, x, ldx, g, b, y, ldy, rows, cols,
                     eps);
  return check_launch("layernorm_bf16");
}

int layer_norm_bf16(const bf16* x, int64_t ldx, const float* g, const float* b, bf16* y, int64_t ldy, int rows,
                    int cols, float eps, hipStream_t stream) {
  if (rows == 0) return QVL_OK;
  const int ch = (cols / 8 + 63) / 64;
  switch (ch) {
    case 1: return launch_ln<1>(x, ldx, g, b, y, ldy, rows, cols, eps, stream);
    case 2: return launch_ln<2>(x, ldx, g, b, y, ldy, rows, cols, eps, stream);
    case 3: return launch_ln<3>(x, ldx, g, b, y, ldy, rows, cols, eps, stream);
    case 4: return launch_ln<4>(x, ldx, g, b, y, ldy, rows, cols, eps, stream);
    case 5: case 6: return launch_ln<6>(x, ldx, g, b, y, ldy, rows, cols, eps, stream);
    case 7: case 8: return launch_ln<8>(x, ldx, g, b, y, ldy, rows, cols, eps, stream);
    case 9: return launch_ln<9>(x, ldx, g, b, y, ldy, rows, cols, eps, stream);
    case 10: case 11: case 12: return launch_ln<12>(x, ldx, g, b, y, ldy, rows, cols, eps, stream);
    case 13: case 14: case 15: case 16: return launch_ln<16>(x, ldx, g, b, y, ldy, rows, cols, eps, stream);
  }
  return set_error(QVL_ERR_UNSUPPORTED, "layer_norm: cols=%d unsupported (max 8192)", cols);
}

// ---------------------------------------------------------------------------------------------
// LayerNorm statistics alone (model.py:384-386) for a LayerNorm folded into the Dense that consumes
// it: stats[row] = (mean, rsqrt(var + eps)) with the same exact two-pass fp32 arithmetic as
// layernorm_bf16_kernel, one wave per row walking rows with the next row's loads in flight. It
// reads the rows once and writes 8 bytes per row (LayerNorm itself also writes the normalised rows).
// ---------------------------------------------------------------------------------------------
template <int CH>
__global__ __launch_bounds__(256) void rowstats_bf16_kernel(const bf16* __restrict__ x, int64_t ldx, int rows,
                                                            int cols, float eps, f32x2* __restrict__ stats) {
  const int lane = threadIdx.x & 63;
  const int stride = gridDim.x * 4;
  const int nch = cols >> 3;
  const float inv_n = 1.0f / (float)cols;
  auto load_row = [&](int r, u32x4* dst) {
    const bf16* xr = x + (int64_t)r * ldx;
#pragma unroll
    for (int i = 0; i < CH; ++i) {
      const int c = lane + 64 * i;
      dst[i] = (c < nch) ? *reinterpret_cast<const u32x4*>(xr + c * 8) : u32x4{0u, 0u, 0u, 0u};
    }
  };
  int row = blockIdx.x * 4 + (threadIdx.x >> 6);
  u32x4 nxt[CH];
  if (row < rows) load_row(row, nxt);
  for (; row < rows; row += stride) {
    float v[CH][8];
    float s = 0.f;
#pragma unroll
    for (int i = 0; i < CH; ++i) {
      const u32x4 w = nxt[i];
      v[i][0] = bf16_lo(w.x); v[i][1] = bf16_hi(w.x); v[i][2] = bf16_lo(w.y); v[i][3] = bf16_hi(w.y);
      v[i][4] = bf16_lo(w.z); v[i][5] = bf16_hi(w.z); v[i][6] = bf16_lo(w.w); v[i][7] = bf16_hi(w.w);
#pragma unroll
      for (int e = 0; e < 8; ++e) s += v[i][e];      // chunks past the row end hold zeros
    }
    if (row + stride < rows) load_row(row + stride, nxt);
    const float mean = wave_sum(s) * inv_n;
    float q = 0.f;
#pragma unroll
    for (int i = 0; i < CH; ++i) {
      const int c = lane + 64 * i;
      if (c < nch) {
#pragma unroll
        for (int e = 0; e < 8; ++e) { const float d = v[i][e] - mean; q += d * d; }
      }
    }
    const float var = wave_sum(q) * inv_n;
    if (lane == 0) stats[row] = f32x2{mean, rsqrtf(var + eps)};
  }
}

template <int CH>
static int launch_rowstats(const bf16* x, int64_t ldx, int rows, int cols, float eps, f32x2* stats,
                           hipStream_t stream) {
  const int grid = std::min((rows + 3) / 4, 4 * gemm_device_cus());
  hipLaunchKernelGGL(rowstats_bf16_kernel<CH>, dim3(grid), dim3(256), 0, stream, x, ldx, rows, cols, eps, stats);
  return check_launch("rowstats_bf16");
}

int row_stats_bf16(const bf16* x, int64_t ldx, int rows, int cols, float eps, f32x2* stats, hipStream_t stream) {
  if (rows == 0) return QVL_OK;
  switch ((cols / 8 + 63) / 64) {
    case 1: return launch_rowstats<1>(x, ldx, rows, cols, eps, stats, stream);
    case 2: return launch_rowstats<2>(x, ldx, rows, cols, eps, stats, stream);
    case 3: return launch_rowstats<3>(x, ldx, rows, cols, eps, stats, stream);
    case 4: return launch_rowstats<4>(x, ldx, rows, cols, eps, stats, stream);
    case 5: case 6: return launch_rowstats<6>(x, ldx, rows, cols, eps, stats, stream);
    case 7: case 8: return launch_rowstats<8>(x, ldx, rows, cols, eps, stats, stream);
    case 9: return launch_rowstats<9>(x, ldx, rows, cols, eps, stats, stream);
    case 10: case 11: case 12: return launch_rowstats<12>(x, ldx, rows, cols, eps, stats, stream);
    case 13: case 14: case 15: case 16: return launch_rowstats<16>(x, ldx, rows, cols, eps, stats, stream);
  }
  return set_error(QVL_ERR_UNSUPPORTED, "row_stats: cols=%d unsupported (max 8192)", cols);
}

// ---------------------------------------------------------------------------------------------
// LayerNorm folded into the next Dense: with xn = (x - mean) r gamma + beta (model.py:387),
//   xn . W[n] = r (x . W'[n]) - r mean c[n] + d[n],  W'[n][k] = bf16(gamma[k] W[n][k]),
//   c[n] = sum_k W'[n][k],  d[n] = sum_k beta[k] W[n][k].
// From the packed kernel w [n_pad][k] (bf16, K contiguous): out [n_pad][k] = W', cd[n] = (c, d);
// padding rows give zeros. One wave per output feature, fp32 sums.
// ---------------------------------------------------------------------------------------------
__global__ __launch_bounds__(256) void fold_ln_weight_kernel(const bf16* __restrict__ w, int k, int n_pad,
                                                             const float* __restrict__ gamma,
                                                             const float* __restrict__ beta, bf16* __restrict__ out,
                                                             f32x2* __restrict__ cd) {
  const int lane = threadIdx.x & 63;
  const int n = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (n >= n_pad) return;
  const bf16* wr = w + (int64_t)n * k;
  bf16* orow = out + (int64_t)n * k;
  float c = 0.f, d = 0.f;
  for (int j = lane * 8; j < k; j += 512) {
    const u32x4 u = *reinterpret_cast<const u32x4*>(wr + j);
    const f32x4 g0 = *reinterpret_cast<const f32x4*>(gamma + j), g1 = *reinterpret_cast<const f32x4*>(gamma + j + 4);
    const f32x4 b0 = *reinterpret_cast<const f32x4*>(beta + j), b1 = *reinterpret_cast<const f32x4*>(beta + j + 4);
    const float wv[8] = {bf16_lo(u.x), bf16_hi(u.x), bf16_lo(u.y), bf16_hi(u.y),
                         bf16_lo(u.z), bf16_hi(u.z), bf16_lo(u.w), bf16_hi(u.w)};
    const float gv[8] = {g0[0], g0[1], g0[2], g0[3], g1[0], g1[1], g1[2], g1[3]};
    const float bv[8] = {b0[0], b0[1], b0[2], b0[3], b1[0], b1[1], b1[2], b1[3]};
    float f[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      f[e] = round_bf16(gv[e] * wv[e]);
      c += f[e];
      d = fmaf(bv[e], wv[e], d);
    }
    *reinterpret_cast<u32x4*>(orow + j) = u32x4{pack_bf16x2(f[0], f[1]), pack_bf16x2(f[2], f[3]),
                                                pack_bf16x2(f[4], f[5]), pack_bf16x2(f[6], f[7])};
  }
  c = wave_sum(c);
  d = wave_sum(d);
  if (lane == 0) cd[n] = f32x2{c, d};
}

int fold_ln_weight_bf16(const bf16* w, int64_t k, int64_t n_pad, const float* gamma, const float* beta, bf16* out,
                        f32x2* cd, hipStream_t stream) {
  if (n_pad == 0) return QVL_OK;
  hipLaunchKernelGGL(fold_ln_weight_kernel, dim3((unsigned)((n_pad + 3) / 4)), dim3(256), 0, stream, w, (int)k,
                     (int)n_pad, gamma, beta, out, cd);
  return check_launch("fold_ln_weight");
}

// ---------------------------------------------------------------------------------------------
// Pos-embed bilinear gather (model.py:751-764): one wave per token, 4 table rows weighted, in
// the reference's bf16 arithmetic: each tap product rounded to bf16, the sum taken left to right
// ((t0 + t1) + t2) + t3 with each partial sum rounded (eager jnp ops, model.py:751-752). Taps
// whose weight is 0 (every tap but one when the grid side equals the table side, e.g. 768-pixel
// images on the 48 x 48 table) are skipped: their products are zeros and leave the sum unchanged
// (up to the sign of a zero sum), and the wave-uniform test saves their row reads.
// ---------------------------------------------------------------------------------------------
__global__ __launch_bounds__(256) void pos_embed_bf16_kernel(const bf16* __restrict__ table,
                                                             const int* __restrict__ idx,
                                                             const float* __restrict__ wts,
                                                             bf16* __restrict__ y, int n_tok, int dim) {
  const int lane = threadIdx.x & 63;
  const int n = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (n >= n_tok) return;
  int ti[4]; float tw[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) { ti[j] = idx[(int64_t)j * n_tok + n]; tw[j] = wts[(int64_t)j * n_tok + n]; }
  for (int c = lane; c < dim / 8; c += 64) {
    float acc[8] = {0, 0, 0, 0, 0, 0, 0, 0};
    bool first = true;                      // wave-uniform
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      if (tw[j] == 0.f) continue;
      const u32x4 w = *reinterpret_cast<const u32x4*>(table + (int64_t)ti[j] * dim + c * 8);
      const float v[8] = {bf16_lo(w.x), bf16_hi(w.x), bf16_lo(w.y), bf16_hi(w.y),
                          bf16_lo(w.z), bf16_hi(w.z), bf16_lo(w.w), bf16_hi(w.w)};
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const float t = round_bf16(tw[j] * v[e]);          // the bf16 product (exact in fp32, rounded once)
        acc[e] = first ? t : round_bf16(acc[e] + t);
      }
      first = false;
    }
    u32x4 o = {pack_bf16x2(acc[0], acc[1]), pack_bf16x2(acc[2], acc[3]), pack_bf16x2(acc[4], acc[5]),
               pack_bf16x2(acc[6], acc[7])};
    *reinterpret_cast<u32x4*>(y + (int64_t)n * dim + c * 8) = o;
  }
}

int pos_embed_bf16(const bf16* table, const int* idx, const float* wts, bf16* y, int n_tok, int dim,
                   hipStream_t stream) {
  if (n_tok == 0) return QVL_OK;
  hipLaunchKernelGGL(pos_embed_bf16_kernel, dim3((n_tok + 3) / 4), dim3(256), 0, stream, table, idx, wts, y,
                     n_tok, dim);
  return check_launch("pos_embed_bf16");
}

// ---------------------------------------------------------------------------------------------
// Rotary table: cs[n, j] = (cos, sin)(pos * inv_freq[j mod hd/4]) with pos = h for j < hd/4,
// w otherwise (model.py:694-698, 821-823); rounded to bf16 values in the bf16 mode.
// ---------------------------------------------------------------------------------------------
struct InvFreq { float v[32]; };

__global__ __launch_bounds__(256) void rotary_table_kernel(const int* __restrict__ pos_hw, int n_tok, int half,
                                                           InvFreq inv, int round16, f32x2* __restrict__ cs) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= (int64_t)n_tok * half) return;
  const int n = (int)(i / half), j = (int)(i % half);
  const int q = half / 2;
  const int pos = pos_hw[2 * n + (j < q ? 0 : 1)];
  const float ang = (float)pos * inv.v[j < q ? j : j - q];
  float c = cosf(ang), s = sinf(ang);
  if (round16) { c = round_bf16(c); s = round_bf16(s); }
  cs[i] = f32x2{c, s};
}

int rotary_table(const int* pos_hw, int n_tok, int head_dim, const float* inv_freq, int round16, f32x2* cs,
                 hipStream_t stream) {
  if (n_tok == 0) return QVL_OK;
  InvFreq inv{};
  for (int j = 0; j < head_dim / 4; ++j) inv.v[j] = inv_freq[j];
  const int half = head_dim / 2;
  const int64_t total = (int64_t)n_tok * half;
  hipLaunchKernelGGL(rotary_table_kernel, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, stream, pos_hw,
                     n_tok, half, inv, round16, cs);
  return check_launch("rotary_table");
}

// Per-position rotary table: t[p][j] = bf16 cos | bf16 sin << 16 of p * inv_freq[j], j < head_dim/4:
// the same fp32 angle, cosf / sinf and rounding as rotary_table_kernel, so a token's (cos, sin) of
// dim j equals t[pos_h][j] (j < head_dim/4) or t[pos_w][j - head_dim/4] bit for bit.
__global__ __launch_bounds__(256) void rotary_pos_table_kernel(int n_pos, int q4, InvFreq inv, uint32_t* __restrict__ t) {
  const int i = blockIdx.x * 256 + threadIdx.x;
  if (i >= n_pos * q4) return;
  const int pos = i / q4, j = i % q4;
  const float ang = (float)pos * inv.v[j];
  t[i] = pack_bf16x2(cosf(ang), sinf(ang));
}

int rotary_pos_table(int n_pos, int head_dim, const float* inv_freq, uint32_t* table, hipStream_t stream) {
  if (n_pos == 0) return QVL_OK;
  InvFreq inv{};
  for (int j = 0; j < head_dim / 4; ++j) inv.v[j] = inv_freq[j];
  const int total = n_pos * (head_dim / 4);
  hipLaunchKernelGGL(rotary_pos_table_kernel, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, stream, n_pos,
                     head_dim / 4, inv, table);
  return check_launch("rotary_pos_table");
}

// ---------------------------------------------------------------------------------------------
// fp32 -> bf16 cast (pixel patches, model.py:556 `x.astype(dtype)`), 8 elements per thread.
// ---------------------------------------------------------------------------------------------
__global__ __launch_bounds__(256) void cast_f32_bf16_kernel(const float* __restrict__ x, bf16* __restrict__ y,
                                                            int64_t n) {
  const int64_t i = ((int64_t)blockIdx.x * 256 + threadIdx.x) * 8;
  if (i + 8 <= n) {
    const f32x4 a = *reinterpret_cast<const f32x4*>(x + i);
    const f32x4 b = *reinterpret_cast<const f32x4*>(x + i + 4);
    u32x4 o = {pack_bf16x2(a[0], a[1]), pack_bf16x2(a[2], a[3]), pack_bf16x2(b[0], b[1]), pack_bf16x2(b[2], b[3])};
    *reinterpret_cast<u32x4*>(y + i) = o;
  } else {
    for (int64_t j = i; j < n; ++j) y[j] = (bf16)x[j];
  }
}

int cast_f32_bf16(const float* x, bf16* y, int64_t n, hipStream_t stream) {
  if (n == 0) return QVL_OK;
  const int64_t threads = (n + 7) / 8;
  hipLaunchKernelGGL(cast_f32_bf16_kernel, dim3((unsigned)((threads + 255) / 256)), dim3(256), 0, stream, x, y, n);
  return check_launch("cast_f32_bf16");
}

// ---------------------------------------------------------------------------------------------
// Weight packing: Flax kernel [k_in, n_out] fp32 -> [n_pad, k_pad] bf16, zero padded.
// 64x64 tiles transposed through LDS.
// ---------------------------------------------------------------------------------------------
__global__ __launch_bounds__(256) void pack_weight_kernel(const float* __restrict__ w, int64_t k_in, int64_t n_out,
                                                          int64_t k_pad, bf16* __restrict__ out) {
  __shared__ float t[64][65];
  const int64_t k0 = (int64_t)blockIdx.x * 64, n0 = (int64_t)blockIdx.y * 64;
  for (int i = threadIdx.x; i < 64 * 64; i += 256) {
    const int r = i / 64, c = i % 64;   // r: k, c: n
    const int64_t k = k0 + r, n = n0 + c;
    t[r][c] = (k < k_in && n < n_out) ? w[k * n_out + n] : 0.f;
  }
  __syncthreads();
  for (int i = threadIdx.x; i < 64 * 64; i += 256) {
    const int r = i / 64, c = i % 64;   // r: n, c: k
    out[(n0 + r) * k_pad + k0 + c] = (bf16)t[c][r];
  }
}

int pack_weight_bf16(const float* w, int64_t k_in, int64_t n_out, bf16* out, hipStream_t stream) {
  const int64_t k_pad = round_up(k_in, 64), n_pad = round_up(n_out, 64);
  hipLaunchKernelGGL(pack_weight_kernel, dim3((unsigned)(k_pad / 64), (unsigned)(n_pad / 64)), dim3(256), 0, stream,
                     w, k_in, n_out, k_pad, out);
  return check_launch("pack_weight");
}

}  // namespace qvl
