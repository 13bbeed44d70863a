// Packed varlen (cu_seqlens) vision attention for gfx950: block-diagonal, non-causal softmax
// attention per segment (model.py:585-600), bf16 MFMA with fp32 online softmax.
//
// Operand layouts (produced by the qkv GEMM's rotary epilogue or by `attn_relayout_kernel`):
//   Q [H][Np][64]  rotated, pre-multiplied by head_dim^-0.5 * log2(e)  (scores land in log2 units)
//   K [H][Np][64]  rotated
//   Vt[H][64][Np]  V transposed (token axis contiguous)
// Rows [n_tokens, Np) are zero.
//
// Each workgroup (4 waves) owns one 128-query tile of one segment and one head; each wave owns
// 32 queries. The kernel computes S^T = K Q^T with v_mfma_f32_32x32x16_bf16, so a lane holds one
// query and 16 keys of a 32-key block: the softmax row statistics are in-register except for one
// exchange with the partner lane (lane ^ 32). The MFMA's C operand is preloaded with -m (the
// running row max), so the accumulator already holds s - m and p = exp2(acc) costs one
// instruction per score. The running max is only raised when a tile's partial row sum shows
// growth beyond 2^64 (or on the first tile): exp2 of a stale max stays finite and the result is
// unchanged because softmax is shift-invariant; every raise rescales O and l exactly.
// P (bf16) is then the B operand of O^T += V^T P^T as it sits in registers; the V^T tile is
// staged in LDS with the matching key permutation (middle 4-key quads of each 16-key group
// swapped) so each lane reads its 8 keys as one 16-byte chunk.
#include <math.h>
#include "qvl_kernels.h"

namespace qvl {

constexpr int kAttnBM = 128;   // queries per workgroup
constexpr int kAttnBN = 64;    // keys per K/V tile
constexpr int kHD = 64;

__device__ __forceinline__ int k_off(int row, int chunk) { return row * kHD + ((chunk ^ (row & 7)) << 3); }
__device__ __forceinline__ int v_off(int d, int chunk) { return d * kAttnBN + ((chunk ^ (d & 7)) << 3); }

__global__ __launch_bounds__(256, 2) void attn_fwd_hd64_kernel(
    const bf16* __restrict__ Q, const bf16* __restrict__ K, const bf16* __restrict__ Vt,
    const int* __restrict__ tiles, int Np, int H, bf16* __restrict__ O, int64_t ldo) {
  __shared__ __attribute__((aligned(16))) bf16 sK[2][kAttnBN * kHD];
  __shared__ __attribute__((aligned(16))) bf16 sV[2][kHD * kAttnBN];

  const int tile = blockIdx.x, head = blockIdx.y;
  const int seg_s = tiles[3 * tile], seg_e = tiles[3 * tile + 1], q0 = tiles[3 * tile + 2];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int l32 = lane & 31, hh = lane >> 5;

  const size_t head_elems = (size_t)Np * kHD;
  const bf16* Qh = Q + head * head_elems;
  const bf16* Kh = K + head * head_elems;
  const bf16* Vh = Vt + head * head_elems;
  const __amdgpu_buffer_rsrc_t rq = make_rsrc(Qh, (uint32_t)(head_elems * 2));
  const __amdgpu_buffer_rsrc_t rk = make_rsrc(Kh, (uint32_t)(head_elems * 2));
  const __amdgpu_buffer_rsrc_t rv = make_rsrc(Vh, (uint32_t)(head_elems * 2));

  // Q fragments (B operand of S^T = K Q^T): query row qrow, dims [16ks + 8hh, +8).
  const int qrow = q0 + wave * 32 + l32;
  bf16x8 qf[4];
#pragma unroll
  for (int ks = 0; ks < 4; ++ks)
    qf[ks] = __builtin_bit_cast(bf16x8, buf_load16(rq, (uint32_t)(((int64_t)qrow * kHD + ks * 16 + hh * 8) * 2)));

  // K/V staging: 4 chunks of 16 bytes per thread per tile (2 of K, 2 of V^T).
  u32x4 stg[4];
  auto load_tile = [&](int kb) {
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const int c = i * 256 + tid;
      const int row = c >> 3, ch = c & 7;
      stg[i] = buf_load16(rk, (uint32_t)(((int64_t)(kb + row) * kHD + ch * 8) * 2));
      stg[2 + i] = buf_load16(rv, (uint32_t)(((int64_t)row * Np + kb + ch * 8) * 2));
    }
  };
  auto store_tile = [&](int buf) {
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const int c = i * 256 + tid;
      const int row = c >> 3, ch = c & 7;
      *reinterpret_cast<u32x4*>(&sK[buf][k_off(row, ch)]) = stg[i];
      // V^T row `row` (= d), keys [8ch, 8ch+8): quads go to positions that make each lane's
      // 8 PV keys contiguous. Group g = ch/2; even ch: keys 16g+0..3 -> 16g+0..3,
      // 16g+4..7 -> 16g+8..11; odd ch: 16g+8..11 -> 16g+4..7, 16g+12..15 -> 16g+12..15.
      const int g = ch >> 1, odd = ch & 1;
      const u32x4 v = stg[2 + i];
      bf16* base = &sV[buf][0];
      *reinterpret_cast<u32x2*>(base + v_off(row, 2 * g) + 4 * odd) = u32x2{v.x, v.y};
      *reinterpret_cast<u32x2*>(base + v_off(row, 2 * g + 1) + 4 * odd) = u32x2{v.z, v.w};
    }
  };

  f32x16 oacc[2] = {f32x16{}, f32x16{}};
  float m_run = 0.f, l_run = 0.f;
  f32x16 negm = f32x16{};

  const int n_kt = (seg_e - seg_s + kAttnBN - 1) / kAttnBN;
  load_tile(seg_s);
  store_tile(0);
  __syncthreads();

  for (int it = 0; it < n_kt; ++it) {
    const int cur = it & 1;
    const int kb = seg_s + it * kAttnBN;
    if (it + 1 < n_kt) load_tile(kb + kAttnBN);

    // S^T blocks: keys [32b, 32b+32) of this tile, C = -m.
    f32x16 s[2];
#pragma unroll
    for (int b = 0; b < 2; ++b) {
      s[b] = negm;
#pragma unroll
      for (int ks = 0; ks < 4; ++ks) {
        const bf16x8 kf = *reinterpret_cast<const bf16x8*>(&sK[cur][k_off(b * 32 + l32, ks * 2 + hh)]);
        s[b] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(kf, qf[ks], s[b], 0, 0, 0);
      }
    }
    // Mask keys past the segment end (last tile only).
    if (kb + kAttnBN > seg_e) {
#pragma unroll
      for (int b = 0; b < 2; ++b)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int key = kb + 32 * b + 8 * (r >> 2) + 4 * hh + (r & 3);
          if (key >= seg_e) s[b][r] = -INFINITY;
        }
    }
    float p[2][16];
    float ts = 0.f;
#pragma unroll
    for (int b = 0; b < 2; ++b)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        p[b][r] = __builtin_amdgcn_exp2f(s[b][r]);
        ts += p[b][r];
      }
    // Raise the running max on the first tile, or when this tile's partial sum got large
    // (covers +inf and NaN-free overflow); wave-uniform branch.
    const bool need = (it == 0) || !(ts <= 0x1p64f);
    if (__builtin_amdgcn_ballot_w64(need) != 0) {
      float mx = -INFINITY;
#pragma unroll
      for (int b = 0; b < 2; ++b)
#pragma unroll
        for (int r = 0; r < 16; ++r) mx = fmaxf(mx, s[b][r]);
      mx = fmaxf(mx, __shfl_xor(mx, 32));
      // s already holds (score - m); raise m by `shift` (first tile: to the tile max).
      const float shift = (it == 0) ? mx : fmaxf(mx, 0.f);
      m_run += shift;
      ts = 0.f;
#pragma unroll
      for (int b = 0; b < 2; ++b)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          p[b][r] = __builtin_amdgcn_exp2f(s[b][r] - shift);
          ts += p[b][r];
        }
      if (it > 0) {   // O and l are still zero on the first tile
        const float alpha = __builtin_amdgcn_exp2f(-shift);
        l_run *= alpha;
#pragma unroll
        for (int r = 0; r < 16; ++r) { oacc[0][r] *= alpha; oacc[1][r] *= alpha; }
      }
#pragma unroll
      for (int r = 0; r < 16; ++r) negm[r] = -m_run;
    }
    l_run += ts;

    // O^T[d][q] += V^T[d][keys] P^T[keys][q]: B operand = 8 P values per lane.
#pragma unroll
    for (int b = 0; b < 2; ++b)
#pragma unroll
      for (int e2 = 0; e2 < 2; ++e2) {
        uint32_t w0 = pack_bf16x2(p[b][8 * e2 + 0], p[b][8 * e2 + 1]);
        uint32_t w1 = pack_bf16x2(p[b][8 * e2 + 2], p[b][8 * e2 + 3]);
        uint32_t w2 = pack_bf16x2(p[b][8 * e2 + 4], p[b][8 * e2 + 5]);
        uint32_t w3 = pack_bf16x2(p[b][8 * e2 + 6], p[b][8 * e2 + 7]);
        const bf16x8 pf = __builtin_bit_cast(bf16x8, u32x4{w0, w1, w2, w3});
        const int g = 2 * b + e2;   // 16-key group within the tile
#pragma unroll
        for (int db = 0; db < 2; ++db) {
          const bf16x8 vf = *reinterpret_cast<const bf16x8*>(&sV[cur][v_off(db * 32 + l32, 2 * g + hh)]);
          oacc[db] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(vf, pf, oacc[db], 0, 0, 0);
        }
      }

    if (it + 1 < n_kt) store_tile(cur ^ 1);
    __syncthreads();
  }

  const float l_tot = l_run + __shfl_xor(l_run, 32);
  const float inv = 1.0f / l_tot;
  if (qrow < seg_e) {
    bf16* orow = O + (int64_t)qrow * ldo + head * kHD;
#pragma unroll
    for (int db = 0; db < 2; ++db)
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const int d = db * 32 + 8 * g + 4 * hh;
        u32x2 o = {pack_bf16x2(oacc[db][4 * g] * inv, oacc[db][4 * g + 1] * inv),
                   pack_bf16x2(oacc[db][4 * g + 2] * inv, oacc[db][4 * g + 3] * inv)};
        *reinterpret_cast<u32x2*>(orow + d) = o;
      }
  }
}

// Relayout for the standalone attention entry: q/k/v [N, H*hd] (row stride ld) -> rotated,
// scaled Q / rotated K [H][Np][64] and V^T [H][64][Np]; rows [N, Np) zero-filled.
// One workgroup = 64 tokens of one head.
__global__ __launch_bounds__(256) void attn_relayout_hd64_kernel(
    const bf16* __restrict__ q, const bf16* __restrict__ k, const bf16* __restrict__ v, int64_t ld,
    const f32x2* __restrict__ cs, int N, int Np, float qscale,
    bf16* __restrict__ Qo, bf16* __restrict__ Ko, bf16* __restrict__ Vto) {
  __shared__ bf16 tv[64][kHD + 2];
  const int n0 = blockIdx.x * 64, head = blockIdx.y, tid = threadIdx.x;
  // rotary pairs: 64 tokens x 32 pairs per tensor
  for (int idx = tid; idx < 64 * 32; idx += 256) {
    const int t = idx >> 5, j = idx & 31, n = n0 + t;
    if (n >= Np) continue;
    float q1 = 0.f, q2 = 0.f, k1 = 0.f, k2 = 0.f;
    if (n < N) {
      const f32x2 c = cs[(int64_t)n * 32 + j];
      const int64_t base = (int64_t)n * ld + head * kHD;
      const float a1 = (float)q[base + j], a2 = (float)q[base + j + 32];
      const float b1 = (float)k[base + j], b2 = (float)k[base + j + 32];
      q1 = (a1 * c.x - a2 * c.y) * qscale; q2 = (a2 * c.x + a1 * c.y) * qscale;
      k1 = b1 * c.x - b2 * c.y; k2 = b2 * c.x + b1 * c.y;
    }
    bf16* qd = Qo + ((int64_t)head * Np + n) * kHD;
    bf16* kd = Ko + ((int64_t)head * Np + n) * kHD;
    qd[j] = (bf16)q1; qd[j + 32] = (bf16)q2;
    kd[j] = (bf16)k1; kd[j + 32] = (bf16)k2;
  }
  for (int idx = tid; idx < 64 * kHD; idx += 256) {
    const int t = idx / kHD, d = idx % kHD, n = n0 + t;
    tv[t][d] = (n < N) ? v[(int64_t)n * ld + head * kHD + d] : (bf16)0.f;
  }
  __syncthreads();
  for (int idx = tid; idx < 64 * kHD; idx += 256) {
    const int d = idx / 64, t = idx % 64, n = n0 + t;
    if (n < Np) Vto[((int64_t)head * kHD + d) * Np + n] = tv[t][d];
  }
}

int attention_hd64(const bf16* Qb, const bf16* Kb, const bf16* Vtb, const int* d_tiles, int64_t n_tiles,
                   int Np, int H, bf16* out, int64_t ldo, hipStream_t stream) {
  if (n_tiles == 0) return QVL_OK;
  hipLaunchKernelGGL(attn_fwd_hd64_kernel, dim3((unsigned)n_tiles, (unsigned)H), dim3(256), 0, stream,
                     Qb, Kb, Vtb, d_tiles, Np, H, out, ldo);
  return check_launch("attn_fwd_hd64");
}

int attention_relayout_hd64(const bf16* q, const bf16* k, const bf16* v, int64_t ld, const f32x2* cs, int N,
                            int Np, int H, float qscale, bf16* Qo, bf16* Ko, bf16* Vto, hipStream_t stream) {
  hipLaunchKernelGGL(attn_relayout_hd64_kernel, dim3((unsigned)(Np / 64), (unsigned)H), dim3(256), 0, stream,
                     q, k, v, ld, cs, N, Np, qscale, Qo, Ko, Vto);
  return check_launch("attn_relayout_hd64");
}

}  // namespace qvl
