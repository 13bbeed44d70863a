// fp32 path of the vision tower (the reference's default dtype, model.py `dtype=jnp.float32`):
// every op computes and stores fp32, so the tower matches the reference's fp32 CPU path to
// rounding-order differences. Dense layers and attention run on v_mfma_f32_32x32x2_f32
// (2048 fp32 MACs per instruction, 32 lanes x 2 k-slots per operand); LayerNorm, pos-embed,
// rotary + head-major relayout and weight packing are the fp32 counterparts of the bf16 kernels.
#include <math.h>

#include <algorithm>

#include "qvl_kernels.h"

namespace qvl {

__device__ __forceinline__ f32x16 mfma_f32(float a, float b, f32x16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x2f32(a, b, c, 0, 0, 0);
}

// ---------------------------------------------------------------------------------------------
// GEMM y[M, N] = epi(x[M, K] . W[N, K]^T + bias), fp32. 128 x 128 tiles, 4 waves (2 x 2) of
// 64 x 64 (2 x 2 blocks of 32 x 32). K staged 32 at a time through two LDS stages (registers ->
// LDS), rows of 128 bytes with the 16-byte chunk XOR-swizzled by (row / 2) % 8. MFMA k-slot
// mapping: step kk of a 32-wide k tile takes k = kk for lanes 0-31 and k = 16 + kk for lanes
// 32-63, so each lane's operands are 16 consecutive floats of its row (four 16-byte reads).
// As in the bf16 GEMM, A = weights and B = activations: a lane's accumulator holds one token and
// runs of 4 consecutive features, stored as 16-byte pieces.
// ---------------------------------------------------------------------------------------------
constexpr int kF32Tile = 128, kF32BK = 32;

__device__ __forceinline__ int f32_lds_off(int row, int chunk) { return row * kF32BK + ((chunk ^ ((row >> 1) & 7)) << 2); }

template <int EPI>
__global__ __launch_bounds__(256) void gemm_f32_kernel(GemmF32Params p) {
  __shared__ __attribute__((aligned(16))) float sm[2][2][kF32Tile * kF32BK];   // [stage][x | w] 64 KB
  const int tiles_n = (p.N + kF32Tile - 1) / kF32Tile;
  const int tiles = ((p.M + kF32Tile - 1) / kF32Tile) * tiles_n;
  // split-K: the units of one K part are consecutive, so one XCD's units share operand rows
  const int unit = xcd_remap(blockIdx.x, tiles * p.split);
  const int tile = unit % tiles, part_i = unit / tiles;
  const int m0 = (tile / tiles_n) * kF32Tile, n0 = (tile % tiles_n) * kF32Tile;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave & 1, wn = wave >> 1;
  const int l32 = lane & 31, hh = lane >> 5;

  // Rows past M / past the packed weight rows read as zeros (buffer range); columns past K of x
  // are masked (the packed weights are zero there).
  const __amdgpu_buffer_rsrc_t rx = make_rsrc(p.x, (uint32_t)((int64_t)p.M * p.lda * 4));
  const __amdgpu_buffer_rsrc_t rw = make_rsrc(p.w, (uint32_t)((int64_t)p.n_rows_w * p.ldw * 4));
  u32x4 gx[4], gw[4];
  auto gload = [&](int kt) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int q = tid + 256 * i, r = q >> 3, c = q & 7;
      const int k = kt * kF32BK + c * 4;
      gx[i] = k < p.K ? buf_load16(rx, (uint32_t)(((int64_t)(m0 + r) * p.lda + k) * 4)) : u32x4{0, 0, 0, 0};
      gw[i] = buf_load16(rw, (uint32_t)(((int64_t)(n0 + r) * p.ldw + k) * 4));
    }
  };
  auto sstore = [&](int st) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int q = tid + 256 * i, r = q >> 3, c = q & 7;
      *reinterpret_cast<u32x4*>(&sm[st][0][f32_lds_off(r, c)]) = gx[i];
      *reinterpret_cast<u32x4*>(&sm[st][1][f32_lds_off(r, c)]) = gw[i];
    }
  };

  f32x16 acc[2][2];
#pragma unroll
  for (int a = 0; a < 2; ++a)
#pragma unroll
    for (int b = 0; b < 2; ++b) acc[a][b] = f32x16{};

  const int KT_all = p.Kp / kF32BK;
  const int kt0 = part_i * KT_all / p.split, KT = (part_i + 1) * KT_all / p.split;
  gload(kt0);
  sstore(0);
  __syncthreads();
  for (int kt = kt0; kt < KT; ++kt) {
    const int cur = (kt - kt0) & 1;
    if (kt + 1 < KT) gload(kt + 1);
    f32x4 wf[2][4], xf[2][4];
#pragma unroll
    for (int a = 0; a < 2; ++a)
#pragma unroll
      for (int c = 0; c < 4; ++c)
        wf[a][c] = *reinterpret_cast<const f32x4*>(&sm[cur][1][f32_lds_off(wn * 64 + a * 32 + l32, hh * 4 + c)]);
#pragma unroll
    for (int b = 0; b < 2; ++b)
#pragma unroll
      for (int c = 0; c < 4; ++c)
        xf[b][c] = *reinterpret_cast<const f32x4*>(&sm[cur][0][f32_lds_off(wm * 64 + b * 32 + l32, hh * 4 + c)]);
#pragma unroll
    for (int kk = 0; kk < 16; ++kk)
#pragma unroll
      for (int a = 0; a < 2; ++a)
#pragma unroll
        for (int b = 0; b < 2; ++b) acc[a][b] = mfma_f32(wf[a][kk >> 2][kk & 3], xf[b][kk >> 2][kk & 3], acc[a][b]);
    if (kt + 1 < KT) {
      sstore(cur ^ 1);
      __syncthreads();
    }
  }

  // Epilogue: block (a, b), register r: feature n0 + wn*64 + 32a + 8(r/4) + 4hh + r%4,
  // token m0 + wm*64 + 32b + l32. A K part stores its raw sums instead.
  if (p.split > 1) {
    const int64_t npad = (int64_t)tiles_n * kF32Tile;
    float* dst = p.part + (int64_t)part_i * p.M * npad;
#pragma unroll
    for (int a = 0; a < 2; ++a)
#pragma unroll
      for (int b = 0; b < 2; ++b) {
        const int m = m0 + wm * 64 + b * 32 + l32;
        if (m >= p.M) continue;
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          const int n = n0 + wn * 64 + a * 32 + 8 * g + 4 * hh;
          *reinterpret_cast<f32x4*>(dst + (int64_t)m * npad + n) =
              f32x4{acc[a][b][4 * g], acc[a][b][4 * g + 1], acc[a][b][4 * g + 2], acc[a][b][4 * g + 3]};
        }
      }
    return;
  }
#pragma unroll
  for (int a = 0; a < 2; ++a)
#pragma unroll
    for (int b = 0; b < 2; ++b) {
      const int m = m0 + wm * 64 + b * 32 + l32;
      if (m >= p.M) continue;
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const int n = n0 + wn * 64 + a * 32 + 8 * g + 4 * hh;
        if (n >= p.N) continue;
        const f32x4 bv = *reinterpret_cast<const f32x4*>(p.bias + n);
        f32x4 v;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          v[e] = acc[a][b][4 * g + e] + bv[e];
          if constexpr (EPI == kEpiBiasGelu) v[e] = gelu_tanh(v[e]);
        }
        if constexpr (EPI == kEpiBiasResidual) v += *reinterpret_cast<const f32x4*>(p.res + (int64_t)m * p.ldr + n);
        *reinterpret_cast<f32x4*>(p.y + (int64_t)m * p.ldc + n) = v;
      }
    }
}

// Sums the K parts of a split fp32 GEMM in part order and applies the epilogue, one thread per 4
// consecutive outputs: y = epi(sum_s part[s] + bias).
template <int EPI>
__global__ __launch_bounds__(256) void gemm_f32_reduce_kernel(GemmF32Params p, int64_t npad) {
  const int64_t q = (int64_t)blockIdx.x * 256 + threadIdx.x, quads = (int64_t)p.M * (p.N / 4);
  if (q >= quads) return;
  const int m = (int)(q / (p.N / 4)), n = (int)(q % (p.N / 4)) * 4;
  const float* src = p.part + (int64_t)m * npad + n;
  const int64_t stride = (int64_t)p.M * npad;
  f32x4 v = *reinterpret_cast<const f32x4*>(src);
  for (int s = 1; s < p.split; ++s) v += *reinterpret_cast<const f32x4*>(src + s * stride);
  const f32x4 bv = *reinterpret_cast<const f32x4*>(p.bias + n);
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    v[e] += bv[e];
    if constexpr (EPI == kEpiBiasGelu) v[e] = gelu_tanh(v[e]);
  }
  if constexpr (EPI == kEpiBiasResidual) v += *reinterpret_cast<const f32x4*>(p.res + (int64_t)m * p.ldr + n);
  *reinterpret_cast<f32x4*>(p.y + (int64_t)m * p.ldc + n) = v;
}

// Plan: one 128 x 128 tile per workgroup, two workgroups per CU (64 KB of LDS each). Where the tiles
// fill at most half of those slots and a workspace holds the partials, K is split into up to 8
// parts (each at least 4 k-steps of 32) so the units fill about one round of slots.
int gemm_f32(GemmF32Params p, int epi, hipStream_t stream) {
  const int tiles_n = (p.N + kF32Tile - 1) / kF32Tile;
  const int tiles = ((p.M + kF32Tile - 1) / kF32Tile) * tiles_n;
  if (tiles == 0) return QVL_OK;
  const int slots = 2 * gemm_device_cus();
  const int64_t npad = (int64_t)tiles_n * kF32Tile;
  int split = 1;
  if (p.part && 2 * tiles <= slots) {
    split = std::min(std::min(8, slots / tiles), p.Kp / kF32BK / 4);
    while (split > 1 && (int64_t)split * p.M * npad > p.part_elems) --split;
  }
  p.split = std::max(split, 1);
  const int grid = tiles * p.split;
  switch (epi) {
    case kEpiBias: hipLaunchKernelGGL(gemm_f32_kernel<kEpiBias>, dim3(grid), dim3(256), 0, stream, p); break;
    case kEpiBiasGelu: hipLaunchKernelGGL(gemm_f32_kernel<kEpiBiasGelu>, dim3(grid), dim3(256), 0, stream, p); break;
    case kEpiBiasResidual:
      hipLaunchKernelGGL(gemm_f32_kernel<kEpiBiasResidual>, dim3(grid), dim3(256), 0, stream, p);
      break;
    default: return set_error(QVL_ERR_INVALID_ARG, "gemm_f32: epilogue %d", epi);
  }
  int rc = check_launch("gemm_f32");
  if (rc || p.split == 1) return rc;
  const int64_t blocks = ((int64_t)p.M * (p.N / 4) + 255) / 256;
  switch (epi) {
    case kEpiBias: hipLaunchKernelGGL(gemm_f32_reduce_kernel<kEpiBias>, dim3((unsigned)blocks), dim3(256), 0, stream, p, npad); break;
    case kEpiBiasGelu: hipLaunchKernelGGL(gemm_f32_reduce_kernel<kEpiBiasGelu>, dim3((unsigned)blocks), dim3(256), 0, stream, p, npad); break;
    default: hipLaunchKernelGGL(gemm_f32_reduce_kernel<kEpiBiasResidual>, dim3((unsigned)blocks), dim3(256), 0, stream, p, npad); break;
  }
  return check_launch("gemm_f32_reduce");
}

// ---------------------------------------------------------------------------------------------
// LayerNorm fp32 (model.py:375-388): one wave per row held in registers (CH 16-byte chunks per
// lane), two-pass mean / biased variance, rsqrt(var + eps), affine.
// ---------------------------------------------------------------------------------------------
__device__ __forceinline__ float wave_sum_f32(float v) {
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) v += __shfl_xor(v, o);
  return v;
}

template <int CH>
__global__ __launch_bounds__(256) void layernorm_f32_kernel(const float* __restrict__ x, int64_t ldx,
                                                            const float* __restrict__ gamma,
                                                            const float* __restrict__ beta, float* __restrict__ y,
                                                            int64_t ldy, int rows, int cols, float eps) {
  const int lane = threadIdx.x & 63;
  const int row = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= rows) return;
  const int nch = cols >> 2;
  const float* xr = x + (int64_t)row * ldx;
  f32x4 v[CH];
  float s = 0.f;
#pragma unroll
  for (int i = 0; i < CH; ++i) {
    const int c = lane + 64 * i;
    v[i] = c < nch ? *reinterpret_cast<const f32x4*>(xr + c * 4) : f32x4{};
    s += (v[i][0] + v[i][1]) + (v[i][2] + v[i][3]);
  }
  const float inv_n = 1.0f / (float)cols;
  const float mean = wave_sum_f32(s) * inv_n;
  float q = 0.f;
#pragma unroll
  for (int i = 0; i < CH; ++i) {
    const int c = lane + 64 * i;
    if (c < nch) {
#pragma unroll
      for (int e = 0; e < 4; ++e) { const float d = v[i][e] - mean; q += d * d; }
    }
  }
  const float var = wave_sum_f32(q) * inv_n;
  const float rstd = 1.0f / sqrtf(var + eps);
  float* yr = y + (int64_t)row * ldy;
#pragma unroll
  for (int i = 0; i < CH; ++i) {
    const int c = lane + 64 * i;
    if (c < nch) {
      const f32x4 g = *reinterpret_cast<const f32x4*>(gamma + c * 4);
      const f32x4 b = *reinterpret_cast<const f32x4*>(beta + c * 4);
      f32x4 o;
#pragma unroll
      for (int e = 0; e < 4; ++e) o[e] = (v[i][e] - mean) * rstd * g[e] + b[e];
      *reinterpret_cast<f32x4*>(yr + c * 4) = o;
    }
  }
}

template <int CH>
static int launch_ln_f32(const float* x, int64_t ldx, const float* g, const float* b, float* y, int64_t ldy,
                         int rows, int cols, float eps, hipStream_t stream) {
  hipLaunchKernelGGL(layernorm_f32_kernel<CH>, dim3((rows + 3) / 4), dim3(256), 0, stream, x, ldx, g, b, y, ldy,
                     rows, cols, eps);
  return check_launch("layernorm_f32");
}

int layer_norm_f32(const float* x, int64_t ldx, const float* g, const float* b, float* y, int64_t ldy, int rows,
                   int cols, float eps, hipStream_t stream) {
  if (rows == 0) return QVL_OK;
  const int per_lane = (cols / 4 + 63) / 64;
  if (per_lane <= 4) return launch_ln_f32<4>(x, ldx, g, b, y, ldy, rows, cols, eps, stream);
  if (per_lane <= 8) return launch_ln_f32<8>(x, ldx, g, b, y, ldy, rows, cols, eps, stream);
  if (per_lane <= 18) return launch_ln_f32<18>(x, ldx, g, b, y, ldy, rows, cols, eps, stream);
  if (per_lane <= 32) return launch_ln_f32<32>(x, ldx, g, b, y, ldy, rows, cols, eps, stream);
  return set_error(QVL_ERR_UNSUPPORTED, "layer_norm: cols=%d unsupported (max 8192)", cols);
}

// ---------------------------------------------------------------------------------------------
// Pos-embed fp32 (model.py:750-752): sum over the 4 bilinear taps of table[idx] * w, products
// and sums rounded in the reference's order ((p0 + p1) + p2) + p3.
// ---------------------------------------------------------------------------------------------
__global__ __launch_bounds__(256) void pos_embed_f32_kernel(const float* __restrict__ table,
                                                            const int* __restrict__ idx,
                                                            const float* __restrict__ wts, float* __restrict__ y,
                                                            int n_tok, int dim) {
#pragma clang fp contract(off)   // products and sums rounded separately, as the reference
  const int lane = threadIdx.x & 63;
  const int n = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (n >= n_tok) return;
  int ti[4];
  float tw[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) { ti[j] = idx[(int64_t)j * n_tok + n]; tw[j] = wts[(int64_t)j * n_tok + n]; }
  for (int c = lane; c < dim / 4; c += 64) {
    f32x4 acc{};
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const f32x4 t = *reinterpret_cast<const f32x4*>(table + (int64_t)ti[j] * dim + c * 4);
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const float pr = t[e] * tw[j];
        acc[e] = j == 0 ? pr : acc[e] + pr;
      }
    }
    *reinterpret_cast<f32x4*>(y + (int64_t)n * dim + c * 4) = acc;
  }
}

int pos_embed_f32(const float* table, const int* idx, const float* wts, float* y, int n_tok, int dim,
                  hipStream_t stream) {
  if (n_tok == 0) return QVL_OK;
  hipLaunchKernelGGL(pos_embed_f32_kernel, dim3((n_tok + 3) / 4), dim3(256), 0, stream, table, idx, wts, y, n_tok,
                     dim);
  return check_launch("pos_embed_f32");
}

// ---------------------------------------------------------------------------------------------
// Weight packing fp32: Flax kernel [k_in, n_out] -> [n_pad, k_pad] fp32 (both padded to 64 with
// zeros), 64 x 64 tiles transposed through LDS.
// ---------------------------------------------------------------------------------------------
__global__ __launch_bounds__(256) void pack_weight_f32_kernel(const float* __restrict__ w, int64_t k_in,
                                                              int64_t n_out, int64_t k_pad, float* __restrict__ out) {
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
    out[(n0 + r) * k_pad + k0 + c] = t[c][r];
  }
}

int pack_weight_f32(const float* w, int64_t k_in, int64_t n_out, float* out, hipStream_t stream) {
  const int64_t k_pad = round_up(k_in, 64), n_pad = round_up(n_out, 64);
  hipLaunchKernelGGL(pack_weight_f32_kernel, dim3((unsigned)(k_pad / 64), (unsigned)(n_pad / 64)), dim3(256), 0,
                     stream, w, k_in, n_out, k_pad, out);
  return check_launch("pack_weight_f32");
}

// ---------------------------------------------------------------------------------------------
// Rotary + head-major relayout, fp32 (model.py:579-582): q, k, v are [N, H*hd] column blocks of
// the qkv Dense output (row stride ld). Writes Q [H][Np][hd] (rotated, times qscale), K
// [H][Np][hd] (rotated), V^T [H][vrows][Np] (rows >= hd zero); tokens [N, Np) zero.
// x*cos + rotate_half(x)*sin with each product and the sum rounded separately, as the reference.
// ---------------------------------------------------------------------------------------------
__global__ __launch_bounds__(256) void attn_relayout_f32_kernel(const float* __restrict__ q, const float* __restrict__ k,
                                                                const float* __restrict__ v, int64_t ld,
                                                                const f32x2* __restrict__ cs, int N, int Np, int hd,
                                                                int vrows, float qscale, float* __restrict__ Qo,
                                                                float* __restrict__ Ko, float* __restrict__ Vto) {
#pragma clang fp contract(off)   // x*cos and rotate_half(x)*sin rounded before the sum, as the reference
  const int head = blockIdx.y;
  const int half = hd / 2;
  // rotary part: one thread per (token, j < hd/2)
  for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < (int64_t)Np * half; i += (int64_t)gridDim.x * 256) {
    const int n = (int)(i / half), j = (int)(i % half);
    float q1 = 0.f, q2 = 0.f, k1 = 0.f, k2 = 0.f;
    if (n < N) {
      const f32x2 t = cs[(int64_t)n * half + j];
      const float* qr = q + (int64_t)n * ld + head * hd;
      const float* kr = k + (int64_t)n * ld + head * hd;
      const float a = qr[j], b = qr[j + half], c = kr[j], d = kr[j + half];
      q1 = a * t.x + (-b) * t.y;
      q2 = b * t.x + a * t.y;
      k1 = c * t.x + (-d) * t.y;
      k2 = d * t.x + c * t.y;
    }
    float* qo = Qo + ((int64_t)head * Np + n) * hd;
    float* ko = Ko + ((int64_t)head * Np + n) * hd;
    qo[j] = q1 * qscale; qo[j + half] = q2 * qscale;
    ko[j] = k1; ko[j + half] = k2;
  }
  // V^T: one thread per (row d, token n), token-contiguous stores
  for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < (int64_t)vrows * Np; i += (int64_t)gridDim.x * 256) {
    const int d = (int)(i / Np), n = (int)(i % Np);
    Vto[((int64_t)head * vrows + d) * Np + n] = (d < hd && n < N) ? v[(int64_t)n * ld + head * hd + d] : 0.f;
  }
}

int attention_relayout_f32(const float* q, const float* k, const float* v, int64_t ld, const f32x2* cs, int N, int Np,
                           int H, int hd, int vrows, float qscale, float* Qo, float* Ko, float* Vto,
                           hipStream_t stream) {
  const int64_t work = std::max<int64_t>((int64_t)Np * (hd / 2), (int64_t)vrows * Np);
  const unsigned gx = (unsigned)std::min<int64_t>((work + 255) / 256, 1024);
  hipLaunchKernelGGL(attn_relayout_f32_kernel, dim3(gx, (unsigned)H), dim3(256), 0, stream, q, k, v, ld, cs, N, Np,
                     hd, vrows, qscale, Qo, Ko, Vto);
  return check_launch("attn_relayout_f32");
}

// ---------------------------------------------------------------------------------------------
// Attention fp32 (model.py:585-598 in the fp32 dtype): per work item one 128-query tile of one
// (segment, head), 4 waves x 32 queries, key tiles of 32 staged through LDS (registers ->
// LDS, two stages). S^T = K Q^T on v_mfma_f32_32x32x2_f32 with the k-slot split dims
// [0, hd/2) | [hd/2, hd), so each lane's Q operand is hd/2 consecutive floats held in registers
// and its K operand hd/2 consecutive floats of one LDS row. A lane then holds one query and 16
// keys (8(r/4) + 4hh + r%4) of the tile: exact online softmax in fp32 (max, exp2 of scores
// already in log2 units, rescale), and the probabilities feed the PV MFMA straight from
// registers (step kk pairs the key of register kk in both lane halves with V^T read as 16-byte
// runs of 4 keys). LDS rows are padded by 4 floats: 16 consecutive rows start in 16 distinct
// 16-byte bank groups. Items of a split list past n_whole are key parts (head | part << 12 | parts
// << 20): a part runs its share of the key tiles and stores the unnormalised O, the running max
// and the row sum (log2 units) for attn_combine_kernel.
// ---------------------------------------------------------------------------------------------
template <int HD>
__global__ __launch_bounds__(256) void attn_fwd_f32_kernel(const float* __restrict__ Q, const float* __restrict__ K,
                                                           const float* __restrict__ Vt, const int* __restrict__ items,
                                                           int Np, float* __restrict__ O, int64_t ldo, int n_whole,
                                                           float* __restrict__ part) {
  constexpr int NDB = (HD + 31) / 32, VR = 32 * NDB, KH = HD / 2;
  constexpr int KS = HD + 4, VS = 32 + 4;
  static_assert(HD % 8 == 0, "head_dim");
  __shared__ __attribute__((aligned(16))) float sK[2][32 * KS];
  __shared__ __attribute__((aligned(16))) float sV[2][VR * VS];

  const int item = blockIdx.x;
  const int seg_s = items[4 * item], seg_e = items[4 * item + 1], q0 = items[4 * item + 2];
  const int hraw = items[4 * item + 3];
  const int head = hraw & kAttnHeadMask;
  const int part_i = (hraw >> kAttnSplitShift) & 0xff, parts = (hraw >> kAttnPartsShift) & 0xff;
  if (seg_e <= seg_s || (parts && (!part || item < n_whole))) return;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int l32 = lane & 31, hh = lane >> 5;

  const size_t qk_elems = (size_t)Np * HD;
  const float* Qh = Q + head * qk_elems;
  const float* Kh = K + head * qk_elems;
  const float* Vh = Vt + (size_t)head * VR * Np;
  const __amdgpu_buffer_rsrc_t rq = make_rsrc(Qh, (uint32_t)(qk_elems * 4));
  const int qrow = q0 + wave * 32 + l32;
  f32x4 qf[KH / 4];
#pragma unroll
  for (int i = 0; i < KH / 4; ++i)
    qf[i] = __builtin_bit_cast(f32x4, buf_load16(rq, (uint32_t)(((int64_t)qrow * HD + hh * KH + 4 * i) * 4)));

  // tile staging: K rows (32 keys x HD) and V^T rows (VR x 32 keys), 16-byte chunks
  constexpr int KCH = 32 * HD / 4, VCH = VR * 8;
  constexpr int KPT = (KCH + 255) / 256, VPT = (VCH + 255) / 256;
  f32x4 gk[KPT], gv[VPT];
  auto gload = [&](int kb) {
#pragma unroll
    for (int i = 0; i < KPT; ++i) {
      const int c = tid + 256 * i, r = c / (HD / 4), e = c % (HD / 4);
      const int key = kb + r;
      gk[i] = (c < KCH && key >= seg_s && key < seg_e) ? *reinterpret_cast<const f32x4*>(Kh + (int64_t)key * HD + 4 * e)
                                                       : f32x4{};
    }
#pragma unroll
    for (int i = 0; i < VPT; ++i) {
      const int c = tid + 256 * i, d = c / 8, e = c % 8;
      const int key = kb + 4 * e;                   // kb is a multiple of 4
      if (c < VCH && key >= seg_s && key + 3 < seg_e) {
        gv[i] = *reinterpret_cast<const f32x4*>(Vh + (int64_t)d * Np + key);
      } else {                                      // segment edges: key by key
        gv[i] = f32x4{};
#pragma unroll
        for (int t = 0; t < 4; ++t)
          if (c < VCH && key + t >= seg_s && key + t < seg_e) gv[i][t] = Vh[(int64_t)d * Np + key + t];
      }
    }
  };
  auto sstore = [&](int st) {
#pragma unroll
    for (int i = 0; i < KPT; ++i) {
      const int c = tid + 256 * i, r = c / (HD / 4), e = c % (HD / 4);
      if (c < KCH) *reinterpret_cast<f32x4*>(&sK[st][r * KS + 4 * e]) = gk[i];
    }
#pragma unroll
    for (int i = 0; i < VPT; ++i) {
      const int c = tid + 256 * i, d = c / 8, e = c % 8;
      if (c < VCH) *reinterpret_cast<f32x4*>(&sV[st][d * VS + 4 * e]) = gv[i];
    }
  };

  f32x16 oacc[NDB];
#pragma unroll
  for (int db = 0; db < NDB; ++db) oacc[db] = f32x16{};
  float m_run = -INFINITY, l_run = 0.f;

  const int k_first = seg_s & ~3;                  // 16-byte aligned V^T runs; keys < seg_s masked
  const int n_all = (seg_e - k_first + 31) / 32;
  const int t0 = parts ? n_all * part_i / parts : 0, t1 = parts ? n_all * (part_i + 1) / parts : n_all;
  const int k_begin = k_first + 32 * t0;
  const int n_kt = t1 - t0;
  gload(k_begin);
  sstore(0);
  __syncthreads();
  for (int it = 0; it < n_kt; ++it) {
    const int cur = it & 1;
    const int kb = k_begin + it * 32;
    if (it + 1 < n_kt) gload(kb + 32);
    // S^T[key][query] over hd
    f32x16 s = f32x16{};
    const float* kr = &sK[cur][l32 * KS + hh * KH];
#pragma unroll
    for (int i = 0; i < KH / 4; ++i) {
      const f32x4 kf = *reinterpret_cast<const f32x4*>(kr + 4 * i);
#pragma unroll
      for (int e = 0; e < 4; ++e) s = mfma_f32(kf[e], qf[i][e], s);
    }
    float mx = -INFINITY;
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int key = kb + 8 * (r >> 2) + 4 * hh + (r & 3);
      if (key < seg_s || key >= seg_e) s[r] = -INFINITY;
      mx = fmaxf(mx, s[r]);
    }
    mx = fmaxf(mx, __shfl_xor(mx, 32));
    const float m_new = fmaxf(m_run, mx);
    const float alpha = __builtin_amdgcn_exp2f(m_run - m_new);
    float ls = 0.f;
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      s[r] = __builtin_amdgcn_exp2f(s[r] - m_new);
      ls += s[r];
    }
    ls += __shfl_xor(ls, 32);
    l_run = l_run * alpha + ls;
    m_run = m_new;
#pragma unroll
    for (int db = 0; db < NDB; ++db) {
      oacc[db] *= alpha;
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const f32x4 vf = *reinterpret_cast<const f32x4*>(&sV[cur][(db * 32 + l32) * VS + 8 * g + 4 * hh]);
#pragma unroll
        for (int e = 0; e < 4; ++e) oacc[db] = mfma_f32(vf[e], s[4 * g + e], oacc[db]);
      }
    }
    if (it + 1 < n_kt) {
      sstore(cur ^ 1);
      __syncthreads();
    }
  }

  if (parts) {
    // a key part: unnormalised O^T rows, (m, l) per query, in the layout attn_combine_kernel reads
    if (qrow < seg_e) {
      float* pp = part + (int64_t)(item - n_whole) * attn_partial_floats(HD);
      const int ql = wave * 32 + l32;
#pragma unroll
      for (int db = 0; db < NDB; ++db)
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          const int d = db * 32 + 8 * g + 4 * hh;
          if (d < HD)
            *reinterpret_cast<f32x4*>(pp + ql * HD + d) =
                f32x4{oacc[db][4 * g], oacc[db][4 * g + 1], oacc[db][4 * g + 2], oacc[db][4 * g + 3]};
        }
      if (hh == 0) *reinterpret_cast<f32x2*>(pp + kAttnBM * HD + 2 * ql) = f32x2{m_run, l_run};
    }
    return;
  }
  if (qrow < seg_e) {
    const float inv = 1.0f / l_run;
    float* orow = O + (int64_t)qrow * ldo + head * HD;
#pragma unroll
    for (int db = 0; db < NDB; ++db)
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const int d = db * 32 + 8 * g + 4 * hh;
        if (d < HD) {
          f32x4 o;
#pragma unroll
          for (int e = 0; e < 4; ++e) o[e] = oacc[db][4 * g + e] * inv;
          *reinterpret_cast<f32x4*>(orow + d) = o;
        }
      }
  }
}

int attention_f32(const float* Qb, const float* Kb, const float* Vtb, const int* d_items, int64_t n_items, int Np,
                  int hd, float* out, int64_t ldo, hipStream_t stream, int64_t n_whole, float* part) {
  if (n_items == 0) return QVL_OK;
  if (n_whole < 0) n_whole = n_items;
  if (hd == 64)
    hipLaunchKernelGGL(attn_fwd_f32_kernel<64>, dim3((unsigned)n_items), dim3(256), 0, stream, Qb, Kb, Vtb, d_items,
                       Np, out, ldo, (int)n_whole, part);
  else if (hd == 72)
    hipLaunchKernelGGL(attn_fwd_f32_kernel<72>, dim3((unsigned)n_items), dim3(256), 0, stream, Qb, Kb, Vtb, d_items,
                       Np, out, ldo, (int)n_whole, part);
  else if (hd == 80)
    hipLaunchKernelGGL(attn_fwd_f32_kernel<80>, dim3((unsigned)n_items), dim3(256), 0, stream, Qb, Kb, Vtb, d_items,
                       Np, out, ldo, (int)n_whole, part);
  else
    return set_error(QVL_ERR_UNSUPPORTED, "attention f32: head_dim=%d (supported: 64, 72, 80)", hd);
  const int rc = check_launch("attn_fwd_f32");
  if (rc || n_whole >= n_items || !part) return rc;
  return attention_combine_f32(d_items, n_items, n_whole, part, out, ldo, hd, stream);
}

}  // namespace qvl
