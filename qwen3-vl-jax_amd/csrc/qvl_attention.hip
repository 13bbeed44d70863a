// Packed varlen (cu_seqlens) vision attention for gfx950: block-diagonal, non-causal softmax
// attention per segment (model.py:585-600), bf16 MFMA with fp32 softmax accumulation.
//
// Operand layouts (produced by the qkv GEMM's rotary epilogue or by `attn_relayout_hd64_kernel`):
//   Q [H][Np][64]  rotated, pre-multiplied by head_dim^-0.5 * log2(e)  (scores land in log2 units)
//   K [H][Np][64]  rotated
//   Vt[H][64][Np]  V transposed, token axis contiguous, keys at positions vt_pos(key)
// Rows / positions [n_tokens, Np) are zero.
//
// Each workgroup (4 waves; 8 waves in two key groups on small lists, attn_fwd_hd64_kernel<2>) owns
// one 128-query tile of one segment and one head; each wave owns 32 queries. Key tiles of 64 start
// at the segment start rounded down to 64, so every K / V^T
// tile is 64-aligned and arrives by LDS DMA (16-byte chunks, XOR swizzle folded into the
// source address); only the first and last tiles carry keys outside the segment and they are
// peeled off the steady-state loop, which has no masking.
//
// S^T = K Q^T via v_mfma_f32_32x32x16_bf16: a lane holds one query and 16 keys of a 32-key block.
// Softmax is shift invariant, and with the tower's scores (log2 units) far inside fp32 range the
// kernel applies no shift at all: p = exp2(s) is one instruction per score and P goes to bf16 pairs
// for the PV MFMA (its B operand, straight from registers); there is no running max, no rescale and
// no per-block check in the loop. The row sums come from the matrix cores: per 16-key group one
// v_mfma_f32_16x16x32_bf16 multiplies the same B operand by a selector fragment (rowsum_selector)
// whose rows 0 and 1 sum the bf16 P of the wave's queries 0..15 and 16..31, so the output is the
// convex combination of V rows with the weights the PV MFMA used (the reference normalises by the
// sum of its fp32 weights, model.py:594-595; the difference is bf16 rounding of P, as in the PV
// product itself). After the loop each wave checks its rows: a row sum outside [2^-64, 2^96] or an
// accumulator above 2^120 (inf / NaN included) means the unshifted sum under- or overflowed, and
// that wave recomputes its rows shifted by the exact row max (global loads: a max pass, then the
// sum pass with fp32 sums), which holds for any finite scores. V^T's quad-swapped key layout makes
// each lane's 8 PV keys one 16-byte LDS chunk. Steady-state tiles run one 32-key block at a time
// (S, softmax, PV), so a block's four K and four V^T fragment reads are issued ahead of its MFMAs
// within the 128-register budget of 4 waves/SIMD.
#include <math.h>
#include <type_traits>
#include "qvl_kernels.h"

namespace qvl {

constexpr int kAttnBN = 64;    // keys per K/V tile
constexpr int kHD = 64;

template <int V> using int_c = std::integral_constant<int, V>;


// LDS offsets of (row, 16-byte chunk) in the 128-byte-row K and V^T tiles. The 16-byte chunk is
// XOR-swizzled with (row/2) % 8: a 16-byte LDS read serves 16 lanes per clock over 64 banks (two
// rows' worth), and the 16 rows one such read touches land in 16 distinct bank groups.
__device__ __forceinline__ int k_off(int row, int chunk) { return row * kHD + ((chunk ^ ((row >> 1) & 7)) << 3); }
__device__ __forceinline__ int v_off(int d, int chunk) { return d * kAttnBN + ((chunk ^ ((d >> 1) & 7)) << 3); }

// A operand of v_mfma_f32_16x16x32_bf16 (lane l: row l % 16, k-slots 8 (l / 16) .. +8) with row 0
// one on k-slot groups 0 and 2 and row 1 on groups 1 and 3. The PV B operand read as a 16x16x32 B
// operand (lane l: column l % 16, k-slot group l / 16) holds in groups 0 / 2 the P of queries 0..15
// and in groups 1 / 3 those of queries 16..31 (the same 16 keys), so output rows 0 and 1 of lane n
// accumulate the row sums of queries n and 16 + n.
__device__ __forceinline__ bf16x8 rowsum_selector(int lane) {
  const uint32_t w = ((lane & 15) == ((lane >> 4) & 1)) ? 0x3F803F80u : 0u;
  return __builtin_bit_cast(bf16x8, u32x4{w, w, w, w});
}

// KS = 2: a workgroup of 8 waves in two groups of 4; both groups take the same 128 queries, group g
// the g-th half of the item's key tiles with a ring of its own, and group 1 hands its unnormalised
// O, shift and row sums to group 0 through LDS at the end (O = O0 2^(m0 - m) + O1 2^(m1 - m), the
// same for the sums), so short segments run half the key tiles per wave with no partial buffer
// and no second launch. Both groups pass the same number of barriers: a group with one tile
// fewer adds one.
template <int KS>
__global__ __launch_bounds__(256 * KS, 4) void attn_fwd_hd64_kernel(
    const bf16* __restrict__ Q, const bf16* __restrict__ K, const bf16* __restrict__ Vt,
    const int* __restrict__ tiles, int Np, int H, bf16* __restrict__ O, int64_t ldo, int n_whole,
    float* __restrict__ part) {
  static_assert(KS == 1 || KS == 2, "one or two key groups");
  constexpr int kStage = 2 * kAttnBN * kHD;   // elements per stage: K [64][64] then V^T [64][64]
  __shared__ __attribute__((aligned(16))) bf16 smem_all[KS * 2 * kStage];

  // Work item: (segment start, segment end, first query, head [| part, parts]); empty items pad
  // short queues.
  const int item = blockIdx.x;
  const int seg_s = tiles[4 * item], seg_e = tiles[4 * item + 1], q0 = tiles[4 * item + 2];
  const int hraw = tiles[4 * item + 3];
  const int head = hraw & kAttnHeadMask;
  const int part_i = (hraw >> kAttnSplitShift) & 0xff, parts = (hraw >> kAttnPartsShift) & 0xff;
  // parts live after the whole items and need the partial buffer
  if (seg_e <= seg_s || (parts && (!part || item < n_whole))) return;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave_all = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int grp = KS == 2 ? wave_all >> 2 : 0, wave = KS == 2 ? wave_all & 3 : wave_all;   // key group, wave in it
  const int l32 = lane & 31, hh = lane >> 5;
  bf16* const smem = smem_all + grp * 2 * kStage;

  const size_t head_elems = (size_t)Np * kHD;
  const __amdgpu_buffer_rsrc_t rq = make_rsrc(Q + head * head_elems, (uint32_t)(head_elems * 2));

  // Q fragments (B operand of S^T = K Q^T): query row qrow, dims [16ks + 8hh, +8).
  const int qrow = q0 + wave * 32 + l32;
  bf16x8 qf[4];
#pragma unroll
  for (int ks = 0; ks < 4; ++ks)
    qf[ks] = __builtin_bit_cast(bf16x8, buf_load16(rq, (uint32_t)(((int64_t)qrow * kHD + ks * 16 + hh * 8) * 2)));

  // K / V^T tile DMA: each wave fills rows [8w, 8w+8) and [32 + 8w, 32 + 8w + 8) of both tiles
  // (1 KB per instruction). Lane j lands in row r = R0 + j/8 at physical chunk j%8 and fetches the
  // logical chunk the read swizzle maps there; (r/2)%8 does not depend on the 32-row half.
  const int drow = wave * 8 + (lane >> 3);
  const int lch = (lane & 7) ^ ((drow >> 1) & 7);
  const u32x4 rk = rsrc_words(K + head * head_elems, (uint32_t)(head_elems * 2));
  const u32x4 rv = rsrc_words(Vt + head * head_elems, (uint32_t)(head_elems * 2));
  const uint32_t kv_lane = (uint32_t)((drow * kHD + lch * 8) * 2);
  const uint32_t vv_lane = (uint32_t)(((int64_t)drow * Np + lch * 8) * 2);
  const uint32_t lds0 = lds_addr_of(smem);
  auto dma_tile = [&](int kb, int stage) {
    const uint32_t kl = lds0 + stage * kStage * 2, vl = kl + kAttnBN * kHD * 2;
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      dma16(rk, kv_lane, (uint32_t)((kb + 32 * i) * kHD * 2), kl + (32 * i + wave * 8) * kHD * 2);
      dma16(rv, vv_lane, (uint32_t)(((int64_t)32 * i * Np + kb) * 2), vl + (32 * i + wave * 8) * kAttnBN * 2);
    }
  };
  // Fragment reads; with a compile-time stage every address is a per-lane base plus an immediate.
  auto k_frag = [&](int stage, int b, int ks) {
    return *reinterpret_cast<const bf16x8*>(&smem[stage * kStage + k_off(b * 32 + l32, ks * 2 + hh)]);
  };
  auto v_frag = [&](int stage, int db, int g) {
    return *reinterpret_cast<const bf16x8*>(&smem[stage * kStage + kAttnBN * kHD + v_off(db * 32 + l32, 2 * g + hh)]);
  };

  f32x16 oacc[2] = {f32x16{}, f32x16{}};
  f32x4 lacc = {0.f, 0.f, 0.f, 0.f};   // row sums: lane n holds queries n (element 0) and 16 + n (1)
  const bf16x8 ones = rowsum_selector(lane);
  float l_run = 0.f;   // the exact path's fp32 row-sum share (this lane's 8 keys of every 16)
  float m_run = 0.f;   // the shift of the scores: 0 on the main path, the exact row max on the exact path

  // Key tiles of 64 from the segment start rounded down to 64; a part of a split item takes its
  // share [t0, t1) of them.
  const int n_all = (seg_e - (seg_s & ~(kAttnBN - 1)) + kAttnBN - 1) / kAttnBN;
  const int t0p = parts ? n_all * part_i / parts : 0, t1 = parts ? n_all * (part_i + 1) / parts : n_all;
  // with two key groups: group 0 the first ceil(half) of them, group 1 the rest (possibly none)
  const int n_steps = KS == 2 ? (t1 - t0p + 1) / 2 : t1 - t0p;
  const int t0 = t0p + grp * n_steps;
  const int n_kt = grp ? t1 - t0 : n_steps;
  const int k_begin = (seg_s & ~(kAttnBN - 1)) + t0 * kAttnBN;

  // keys outside [seg_s, seg_e) -> -inf. Element r of a lane is key kb + 32 b + 4 hh + 8 (r / 4) + r % 4:
  // one unsigned range test against the lane's bounds per element (the offsets are constants).
  auto mask_block = [&](f32x16& s, int kb, int b) {
    const int lo = seg_s - (kb + 32 * b + 4 * hh);
    const uint32_t span = (uint32_t)(seg_e - seg_s);
#pragma unroll
    for (int r = 0; r < 16; ++r)
      if ((uint32_t)(8 * (r >> 2) + (r & 3) - lo) >= span) s[r] = -INFINITY;
  };
  // p = exp2(s - sh) as bf16 pairs, fp32 row-sum share
  auto exp_pack = [&](const f32x16& s, float sh, uint32_t (&pk)[8]) {
    float ta = 0.f, tb = 0.f;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const float e0 = __builtin_amdgcn_exp2f(s[2 * j] - sh), e1 = __builtin_amdgcn_exp2f(s[2 * j + 1] - sh);
      pk[j] = pack_bf16x2(e0, e1);
      ta = j ? ta + e0 : e0;
      tb = j ? tb + e1 : e1;
    }
    l_run += ta + tb;
  };
  // O^T[d][q] += V^T[d][keys] P^T[keys][q]: B operand = 8 P values per lane; the row sums beside.
  auto pv = [&](const bf16x8 (&vf)[4], const uint32_t (&pk)[8]) {
#pragma unroll
    for (int e2 = 0; e2 < 2; ++e2) {
      const bf16x8 pf = __builtin_bit_cast(bf16x8, u32x4{pk[4 * e2], pk[4 * e2 + 1], pk[4 * e2 + 2], pk[4 * e2 + 3]});
#pragma unroll
      for (int db = 0; db < 2; ++db)
        oacc[db] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(vf[2 * e2 + db], pf, oacc[db], 0, 0, 0);
      lacc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ones, pf, lacc, 0, 0, 0);
    }
  };
  auto exp_only = [&](const f32x16& s, uint32_t (&pk)[8]) {   // p = exp2(s) as bf16 pairs
#pragma unroll
    for (int j = 0; j < 8; ++j) pk[j] = pack_bf16x2(__builtin_amdgcn_exp2f(s[2 * j]), __builtin_amdgcn_exp2f(s[2 * j + 1]));
  };

  // One key tile in LDS stage ST; EDGE masks keys outside the segment (first and last tiles).
  auto step = [&](auto edge_tag, auto stage_tag, int it) {
    constexpr bool EDGE = decltype(edge_tag)::value;
    constexpr int ST = decltype(stage_tag)::value;
    const int kb = k_begin + it * kAttnBN;
    if (it + 1 < n_kt) dma_tile(kb + kAttnBN, ST ^ 1);
    // A wave issuing MFMAs takes issue priority (s_setprio) over the SIMD's other waves, which are
    // then in their softmax VALU work (same-box A/B: -1.5 % at config 2).
#pragma unroll
    for (int b = 0; b < 2; ++b) {
      if constexpr (EDGE) {
        // first / last tile (once per item): fragments are read next to their MFMAs, so the mask's
        // temporaries fit the register budget without spills
        __builtin_amdgcn_s_setprio(1);
        f32x16 s = f32x16{};
#pragma unroll
        for (int ks = 0; ks < 4; ++ks) s = __builtin_amdgcn_mfma_f32_32x32x16_bf16(k_frag(ST, b, ks), qf[ks], s, 0, 0, 0);
        __builtin_amdgcn_s_setprio(0);
        mask_block(s, kb, b);
        uint32_t pk[8];
        exp_only(s, pk);
        __builtin_amdgcn_s_setprio(1);
#pragma unroll
        for (int e2 = 0; e2 < 2; ++e2) {
          const bf16x8 pf = __builtin_bit_cast(bf16x8, u32x4{pk[4 * e2], pk[4 * e2 + 1], pk[4 * e2 + 2], pk[4 * e2 + 3]});
#pragma unroll
          for (int db = 0; db < 2; ++db)
            oacc[db] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(v_frag(ST, db, 2 * b + e2), pf, oacc[db], 0, 0, 0);
          lacc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ones, pf, lacc, 0, 0, 0);
        }
        __builtin_amdgcn_s_setprio(0);
      } else {
        // steady state: the block's K and V^T fragment reads are in flight ahead of its MFMAs
        bf16x8 kf[4];
#pragma unroll
        for (int ks = 0; ks < 4; ++ks) kf[ks] = k_frag(ST, b, ks);
        __builtin_amdgcn_s_setprio(1);
        f32x16 s = f32x16{};
#pragma unroll
        for (int ks = 0; ks < 4; ++ks) s = __builtin_amdgcn_mfma_f32_32x32x16_bf16(kf[ks], qf[ks], s, 0, 0, 0);
        bf16x8 vf[4];
#pragma unroll
        for (int e2 = 0; e2 < 2; ++e2)
#pragma unroll
          for (int db = 0; db < 2; ++db) vf[2 * e2 + db] = v_frag(ST, db, 2 * b + e2);
        __builtin_amdgcn_s_setprio(0);
        uint32_t pk[8];
        exp_only(s, pk);
        __builtin_amdgcn_s_setprio(1);
        pv(vf, pk);
        __builtin_amdgcn_s_setprio(0);
      }
    }
    wait_dma();
    __syncthreads();
  };

  if (KS == 1 || n_kt > 0) dma_tile(k_begin, 0);
  wait_dma();
  __syncthreads();
  // Tile it sits in stage it % 2: tile 0 (masked), then odd/even pairs so each stage is a constant.
  // Every step ends in one barrier: n_kt of them, plus n_steps - n_kt for a group with fewer tiles.
  if (KS == 1 || n_kt > 0) {
    step(std::true_type{}, int_c<0>{}, 0);
    int it = 1;
    for (; it + 2 < n_kt; it += 2) {
      step(std::false_type{}, int_c<1>{}, it);
      step(std::false_type{}, int_c<0>{}, it + 1);
    }
    if (it == n_kt - 2) {
      step(std::false_type{}, int_c<1>{}, it);
      step(std::true_type{}, int_c<0>{}, it + 1);
    } else if (it == n_kt - 1) {
      step(std::true_type{}, int_c<1>{}, it);
    }
  }
  if constexpr (KS == 2) {
    for (int s = n_kt; s < n_steps; ++s) __syncthreads();
  }

  const float la = __shfl(lacc[0], lane & 15), lb = __shfl(lacc[1], lane & 15);
  float l_tot = (l32 & 16) ? lb : la;   // lanes q and q + 32 both hold query q's sum
  // Every accumulator finite and at most 2^120: one comparison each, which inf and NaN fail (a
  // running fmaxf would skip a NaN, e.g. the +inf + -inf of an overflowed PV sum).
  bool o_ok = true;
#pragma unroll
  for (int r = 0; r < 16; ++r) o_ok = o_ok & (fabsf(oacc[0][r]) <= 0x1p120f) & (fabsf(oacc[1][r]) <= 0x1p120f);
  if (KS == 2 && n_kt == 0) {
    m_run = -INFINITY;   // an empty key group (KS = 2, one tile): weight 0 in the combine below
  } else if (__builtin_amdgcn_ballot_w64(!(l_tot >= 0x1p-64f && l_tot <= 0x1p96f) || !o_ok) != 0) {
    // Some row's sum of 2^s left [2^-64, 2^96] (or O grew past 2^120, or anything overflowed):
    // recompute this wave's rows shifted by the exact row max, reading K and V^T from global
    // memory (the other waves may be done).
    const __amdgpu_buffer_rsrc_t rkg = make_rsrc(K + head * head_elems, (uint32_t)(head_elems * 2));
    const __amdgpu_buffer_rsrc_t rvg = make_rsrc(Vt + head * head_elems, (uint32_t)(head_elems * 2));
    bf16x8 qg[4];   // reloaded: the loop's fragments are not kept live past it
#pragma unroll
    for (int ks = 0; ks < 4; ++ks)
      qg[ks] = __builtin_bit_cast(bf16x8, buf_load16(rq, (uint32_t)(((int64_t)qrow * kHD + ks * 16 + hh * 8) * 2)));
    auto scores = [&](int kb, int b) {
      f32x16 s = f32x16{};
#pragma unroll
      for (int ks = 0; ks < 4; ++ks) {
        const bf16x8 kf = __builtin_bit_cast(
            bf16x8, buf_load16(rkg, (uint32_t)(((int64_t)(kb + 32 * b + l32) * kHD + ks * 16 + hh * 8) * 2)));
        s = __builtin_amdgcn_mfma_f32_32x32x16_bf16(kf, qg[ks], s, 0, 0, 0);
      }
      mask_block(s, kb, b);
      return s;
    };
    float mx = -INFINITY;
    for (int t = 0; t < n_kt; ++t)
#pragma unroll
      for (int b = 0; b < 2; ++b) {
        const f32x16 s = scores(k_begin + t * kAttnBN, b);
#pragma unroll
        for (int r = 0; r < 16; ++r) mx = fmaxf(mx, s[r]);
      }
    m_run = fmaxf(mx, __shfl_xor(mx, 32));
    oacc[0] = f32x16{};
    oacc[1] = f32x16{};
    l_run = 0.f;
    for (int t = 0; t < n_kt; ++t) {
      const int kb = k_begin + t * kAttnBN;
#pragma unroll
      for (int b = 0; b < 2; ++b) {
        uint32_t pk[8];
        exp_pack(scores(kb, b), m_run, pk);
        bf16x8 vf[4];
#pragma unroll
        for (int e2 = 0; e2 < 2; ++e2)
#pragma unroll
          for (int db = 0; db < 2; ++db)
            vf[2 * e2 + db] = __builtin_bit_cast(
                bf16x8, buf_load16(rvg, (uint32_t)(((int64_t)(db * 32 + l32) * Np + kb + (2 * (2 * b + e2) + hh) * 8) * 2)));
        pv(vf, pk);
      }
    }
    l_tot = l_run + __shfl_xor(l_run, 32);
  }

  if constexpr (KS == 2) {
    // Group 1 hands (O, m, l) to the group 0 wave of the same queries through the free rings
    // ([wave][register][lane] floats: consecutive lanes, consecutive banks); group 0 rescales both
    // to the larger shift and adds (the shifts are 0 unless a group took the exact path).
    float* const xo = reinterpret_cast<float*>(smem_all) + wave * (34 * 64);
    if (grp == 1) {
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        xo[r * 64 + lane] = oacc[0][r];
        xo[(16 + r) * 64 + lane] = oacc[1][r];
      }
      xo[32 * 64 + lane] = m_run;
      xo[33 * 64 + lane] = l_tot;
    }
    __syncthreads();
    if (grp == 1) return;
    const float m1 = xo[32 * 64 + lane], l1 = xo[33 * 64 + lane];
    const float m = fmaxf(m_run, m1);
    const float w0 = exp2f(m_run - m), w1 = m1 == -INFINITY ? 0.f : exp2f(m1 - m);
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      oacc[0][r] = oacc[0][r] * w0 + xo[r * 64 + lane] * w1;
      oacc[1][r] = oacc[1][r] * w0 + xo[(16 + r) * 64 + lane] * w1;
    }
    l_tot = l_tot * w0 + l1 * w1;
    m_run = m;
  }

  if (parts) {
    // Part of a split item: unnormalised O^T, m and row sum, for the combine kernel.
    if (qrow < seg_e) {
      float* pp = part + (int64_t)(item - n_whole) * attn_partial_floats(kHD);
      const int ql = wave * 32 + l32;
#pragma unroll
      for (int db = 0; db < 2; ++db)
#pragma unroll
        for (int g = 0; g < 4; ++g)
          *reinterpret_cast<f32x4*>(pp + ql * kHD + db * 32 + 8 * g + 4 * hh) =
              f32x4{oacc[db][4 * g], oacc[db][4 * g + 1], oacc[db][4 * g + 2], oacc[db][4 * g + 3]};
      if (hh == 0) *reinterpret_cast<f32x2*>(pp + kAttnBM * kHD + 2 * ql) = f32x2{m_run, l_tot};
    }
    return;
  }
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

// ---------------------------------------------------------------------------------------------
// head_dim HD = 72 (the 8B tower) or 80: Q/K [H][Np][88] (dims HD..87 zero; the QK MFMAs use dims
// 0..79), V^T [H][HD][Np] (keys at vt_pos). Same work items, unshifted softmax with the exact
// fallback, and block-at-a-time steady state as the hd-64 kernel. K tiles arrive by LDS DMA as
// contiguous 176-byte rows: 11 16-byte chunks, an odd count, so the 16 rows one fragment read touches
// fall on 16 distinct bank groups without a swizzle. V^T tiles arrive as 128-byte rows with the hd-64
// kernel's XOR swizzle; the third 32-row PV block reads LDS rows 64..95, of which the DMA writes rows
// below HD: row HD holds ones, so output row HD accumulates the softmax row sums (no VALU adds for
// them); the rows above it only feed output rows that are not stored (an MFMA output row depends on
// its own A row only).
// ---------------------------------------------------------------------------------------------
constexpr int kQK72 = 88;                  // Q/K row length (elements)
constexpr int kKS72 = 5;                   // QK k-steps (dims 0..79)
constexpr int kNDB72 = 3;                  // 32-row PV blocks (rows 0..95)
constexpr int kKTile72 = kAttnBN * kQK72;  // K tile elements (11 KB)
constexpr int kVTile72 = 96 * kAttnBN;     // V^T tile elements (12 KB)

__device__ __forceinline__ int k72_off(int row, int chunk) { return row * kQK72 + (chunk << 3); }

template <int HD>
__global__ __launch_bounds__(256, 3) void attn_fwd_qk88_kernel(
    const bf16* __restrict__ Q, const bf16* __restrict__ K, const bf16* __restrict__ Vt,
    const int* __restrict__ tiles, int Np, int H, bf16* __restrict__ O, int64_t ldo, int n_whole,
    float* __restrict__ part) {
  __shared__ __attribute__((aligned(16))) bf16 smem[2 * (kKTile72 + kVTile72)];   // [stage][K 64x88 | V^T 96x64]

  const int item = blockIdx.x;
  const int seg_s = tiles[4 * item], seg_e = tiles[4 * item + 1], q0 = tiles[4 * item + 2];
  const int hraw = tiles[4 * item + 3];
  const int head = hraw & kAttnHeadMask;
  const int part_i = (hraw >> kAttnSplitShift) & 0xff, parts = (hraw >> kAttnPartsShift) & 0xff;
  // parts live after the whole items and need the partial buffer
  if (seg_e <= seg_s || (parts && (!part || item < n_whole))) return;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int l32 = lane & 31, hh = lane >> 5;

  static_assert(HD == 72 || HD == 80, "88-element Q/K rows, three 32-row PV blocks");
  const size_t qk_head = (size_t)Np * kQK72, v_head = (size_t)HD * Np;
  const __amdgpu_buffer_rsrc_t rq = make_rsrc(Q + head * qk_head, (uint32_t)(qk_head * 2));
  const int qrow = q0 + wave * 32 + l32;
  bf16x8 qf[kKS72];
#pragma unroll
  for (int ks = 0; ks < kKS72; ++ks)
    qf[ks] = __builtin_bit_cast(bf16x8, buf_load16(rq, (uint32_t)(((int64_t)qrow * kQK72 + ks * 16 + hh * 8) * 2)));

  // Tile DMA, 11 + HD/8 instructions of 1 KB dealt round-robin to the 4 waves: K instructions 0..10
  // copy the tile's 11264 contiguous bytes (lane j -> byte 16j of the kilobyte); V^T instructions
  // 0..HD/8-1 fill rows [8i, 8i+8), lane j in row 8i + j/8 at physical chunk j%8, fetching the
  // logical chunk the read swizzle maps there ((row/2)%8 alternates with the parity of i).
  const u32x4 rk = rsrc_words(K + head * qk_head, (uint32_t)(qk_head * 2));
  const u32x4 rv = rsrc_words(Vt + head * v_head, (uint32_t)(v_head * 2));
  const uint32_t k_lane = (uint32_t)(lane * 16);
  const int vr = lane >> 3;
  const uint32_t v_lane[2] = {(uint32_t)(((int64_t)vr * Np + (((lane & 7) ^ ((vr >> 1) & 7)) << 3)) * 2),
                              (uint32_t)(((int64_t)vr * Np + (((lane & 7) ^ (((vr >> 1) + 4) & 7)) << 3)) * 2)};
  const uint32_t lds0 = lds_addr_of(smem);
  constexpr uint32_t kStageBytes = (kKTile72 + kVTile72) * 2;
  auto dma_tile = [&](int kb, int stage) {
    const uint32_t kl = lds0 + stage * kStageBytes, vl = kl + kKTile72 * 2;
    constexpr int kInstr = 11 + HD / 8;
#pragma unroll
    for (int j = 0; j < (kInstr + 3) / 4; ++j) {
      const int n = wave + 4 * j;             // instruction 0..kInstr-1, wave-uniform
      if (n < 11) {
        dma16(rk, k_lane, (uint32_t)(kb * kQK72 * 2 + n * 1024), kl + n * 1024);
      } else if (kInstr % 4 == 0 || n < kInstr) {   // (72: 20 instructions, 5 per wave, no check)
        const int i = n - 11;                 // V^T rows [8i, 8i+8)
        dma16(rv, v_lane[i & 1], (uint32_t)(((int64_t)8 * i * Np + kb) * 2), vl + 8 * i * kAttnBN * 2);
      }
    }
  };

  f32x16 oacc[kNDB72] = {f32x16{}, f32x16{}, f32x16{}};
  float m_run = 0.f;   // the shift of the scores: 0 on the main path, the exact row max on the exact path

  const int n_all = (seg_e - (seg_s & ~(kAttnBN - 1)) + kAttnBN - 1) / kAttnBN;
  const int t0 = parts ? n_all * part_i / parts : 0, t1 = parts ? n_all * (part_i + 1) / parts : n_all;
  const int k_begin = (seg_s & ~(kAttnBN - 1)) + t0 * kAttnBN;
  const int n_kt = t1 - t0;
  dma_tile(k_begin, 0);
  // Row HD of both V^T stages holds ones (the DMA fills rows 0..HD-1 only): the third PV block then
  // accumulates each query's row sum of the bf16 P in O^T row HD.
  if (tid < 16)
    *reinterpret_cast<u32x4*>(smem + (tid >> 3) * (kKTile72 + kVTile72) + kKTile72 + HD * kAttnBN + (tid & 7) * 8) =
        u32x4{0x3F803F80u, 0x3F803F80u, 0x3F803F80u, 0x3F803F80u};
  wait_dma();
  __syncthreads();

  auto mask_block = [&](f32x16& s, int kb, int b) {
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int key = kb + 32 * b + 8 * (r >> 2) + 4 * hh + (r & 3);
      if (key < seg_s || key >= seg_e) s[r] = -INFINITY;
    }
  };
  auto pv_frags = [&](const bf16x8 (&vf)[2][kNDB72], const uint32_t (&pk)[8]) {
#pragma unroll
    for (int e2 = 0; e2 < 2; ++e2) {
      const bf16x8 pf = __builtin_bit_cast(bf16x8, u32x4{pk[4 * e2], pk[4 * e2 + 1], pk[4 * e2 + 2], pk[4 * e2 + 3]});
#pragma unroll
      for (int db = 0; db < kNDB72; ++db)
        oacc[db] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(vf[e2][db], pf, oacc[db], 0, 0, 0);
    }
  };
  // One key tile in LDS stage ST, one 32-key block at a time; EDGE masks keys outside the segment.
  auto step = [&](auto edge_tag, auto stage_tag, int it) {
    constexpr bool EDGE = decltype(edge_tag)::value;
    constexpr int ST = decltype(stage_tag)::value;
    const int kb = k_begin + it * kAttnBN;
    if (it + 1 < n_kt) dma_tile(kb + kAttnBN, ST ^ 1);
    const bf16* sK = smem + ST * (kKTile72 + kVTile72);
    const bf16* sV = sK + kKTile72;
#pragma unroll
    for (int b = 0; b < 2; ++b) {
      f32x16 s = f32x16{};
#pragma unroll
      for (int ks = 0; ks < kKS72; ++ks) {
        const bf16x8 kf = *reinterpret_cast<const bf16x8*>(&sK[k72_off(b * 32 + l32, ks * 2 + hh)]);
        s = __builtin_amdgcn_mfma_f32_32x32x16_bf16(kf, qf[ks], s, 0, 0, 0);
      }
      if constexpr (EDGE) mask_block(s, kb, b);
      bf16x8 vf[2][kNDB72];
#pragma unroll
      for (int e2 = 0; e2 < 2; ++e2)
#pragma unroll
        for (int db = 0; db < kNDB72; ++db)
          vf[e2][db] = *reinterpret_cast<const bf16x8*>(&sV[v_off(db * 32 + l32, 2 * (2 * b + e2) + hh)]);
      uint32_t pk[8];
#pragma unroll
      for (int j = 0; j < 8; ++j) pk[j] = pack_bf16x2(__builtin_amdgcn_exp2f(s[2 * j]), __builtin_amdgcn_exp2f(s[2 * j + 1]));
      pv_frags(vf, pk);
    }
    wait_dma();
    __syncthreads();
  };
  step(std::true_type{}, int_c<0>{}, 0);
  int it = 1;
  for (; it + 2 < n_kt; it += 2) {
    step(std::false_type{}, int_c<1>{}, it);
    step(std::false_type{}, int_c<0>{}, it + 1);
  }
  if (it == n_kt - 2) {
    step(std::false_type{}, int_c<1>{}, it);
    step(std::true_type{}, int_c<0>{}, it + 1);
  } else if (it == n_kt - 1) {
    step(std::true_type{}, int_c<1>{}, it);
  }

  // O^T row HD is the row sum of query l32: block 2's local row RS = HD - 64 sits in register
  // 4 (RS / 8) + RS % 4 of the lanes with hh = (RS % 8) / 4 (72: register 4, 80: register 8; hh 0)
  constexpr int RS = HD - 64, RS_REG = 4 * (RS / 8) + RS % 4, RS_HH = (RS % 8) / 4;
  const float l_row = oacc[2][RS_REG], l_swap = __shfl_xor(l_row, 32);
  float l_tot = hh == RS_HH ? l_row : l_swap;
  // |O| over the stored rows: block 2 holds output rows 64..HD-1 in registers 0..4 (RS / 8) - 1; its
  // other registers are the row sum (row HD) and rows above it, products of LDS rows the DMA never writes
  // (every accumulator finite and at most 2^120, tested by comparisons as in attn_fwd_hd64_kernel)
  bool o_ok = true;
#pragma unroll
  for (int r = 0; r < 16; ++r) o_ok = o_ok & (fabsf(oacc[0][r]) <= 0x1p120f) & (fabsf(oacc[1][r]) <= 0x1p120f);
#pragma unroll
  for (int r = 0; r < 4 * (RS / 8); ++r) o_ok = o_ok & (fabsf(oacc[2][r]) <= 0x1p120f);
  if (__builtin_amdgcn_ballot_w64(!(l_tot >= 0x1p-64f && l_tot <= 0x1p96f) || !o_ok) != 0) {
    // As in attn_fwd_hd64_kernel: recompute this wave's rows shifted by the exact row max, from
    // global memory; the row sum by fp32 adds (V^T rows past HD - 1 read as zero: one head's range).
    const __amdgpu_buffer_rsrc_t rkg = make_rsrc(K + head * qk_head, (uint32_t)(qk_head * 2));
    const __amdgpu_buffer_rsrc_t rvg = make_rsrc(Vt + head * v_head, (uint32_t)(v_head * 2));
    bf16x8 qg[kKS72];
#pragma unroll
    for (int ks = 0; ks < kKS72; ++ks)
      qg[ks] = __builtin_bit_cast(bf16x8, buf_load16(rq, (uint32_t)(((int64_t)qrow * kQK72 + ks * 16 + hh * 8) * 2)));
    auto scores = [&](int kb, int b) {
      f32x16 s = f32x16{};
#pragma unroll
      for (int ks = 0; ks < kKS72; ++ks) {
        const bf16x8 kf = __builtin_bit_cast(
            bf16x8, buf_load16(rkg, (uint32_t)(((int64_t)(kb + 32 * b + l32) * kQK72 + ks * 16 + hh * 8) * 2)));
        s = __builtin_amdgcn_mfma_f32_32x32x16_bf16(kf, qg[ks], s, 0, 0, 0);
      }
      mask_block(s, kb, b);
      return s;
    };
    float mx = -INFINITY;
    for (int t = 0; t < n_kt; ++t)
#pragma unroll
      for (int b = 0; b < 2; ++b) {
        const f32x16 s = scores(k_begin + t * kAttnBN, b);
#pragma unroll
        for (int r = 0; r < 16; ++r) mx = fmaxf(mx, s[r]);
      }
    m_run = fmaxf(mx, __shfl_xor(mx, 32));
#pragma unroll
    for (int db = 0; db < kNDB72; ++db) oacc[db] = f32x16{};
    float lsum = 0.f;
    for (int t = 0; t < n_kt; ++t) {
      const int kb = k_begin + t * kAttnBN;
#pragma unroll
      for (int b = 0; b < 2; ++b) {
        const f32x16 s = scores(kb, b);
        uint32_t pk[8];
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          const float e0 = __builtin_amdgcn_exp2f(s[2 * j] - m_run), e1 = __builtin_amdgcn_exp2f(s[2 * j + 1] - m_run);
          pk[j] = pack_bf16x2(e0, e1);
          lsum += e0 + e1;
        }
        bf16x8 vf[2][kNDB72];
#pragma unroll
        for (int e2 = 0; e2 < 2; ++e2)
#pragma unroll
          for (int db = 0; db < kNDB72; ++db)
            vf[e2][db] = __builtin_bit_cast(
                bf16x8, buf_load16(rvg, (uint32_t)(((int64_t)(db * 32 + l32) * Np + kb + (2 * (2 * b + e2) + hh) * 8) * 2)));
        pv_frags(vf, pk);
      }
    }
    l_tot = lsum + __shfl_xor(lsum, 32);
  }
  if (parts) {
    if (qrow < seg_e) {
      float* pp = part + (int64_t)(item - n_whole) * attn_partial_floats(HD);
      const int ql = wave * 32 + l32;
#pragma unroll
      for (int db = 0; db < kNDB72; ++db)
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          const int d = db * 32 + 8 * g + 4 * hh;
          if (d >= HD) continue;
          *reinterpret_cast<f32x4*>(pp + ql * HD + d) =
              f32x4{oacc[db][4 * g], oacc[db][4 * g + 1], oacc[db][4 * g + 2], oacc[db][4 * g + 3]};
        }
      if (hh == 0) *reinterpret_cast<f32x2*>(pp + kAttnBM * HD + 2 * ql) = f32x2{m_run, l_tot};
    }
    return;
  }
  const float inv = 1.0f / l_tot;
  if (qrow < seg_e) {
    bf16* orow = O + (int64_t)qrow * ldo + head * HD;
#pragma unroll
    for (int db = 0; db < kNDB72; ++db)
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const int d = db * 32 + 8 * g + 4 * hh;
        if (d >= HD) continue;
        u32x2 o = {pack_bf16x2(oacc[db][4 * g] * inv, oacc[db][4 * g + 1] * inv),
                   pack_bf16x2(oacc[db][4 * g + 2] * inv, oacc[db][4 * g + 3] * inv)};
        *reinterpret_cast<u32x2*>(orow + d) = o;
      }
  }
}


// ---------------------------------------------------------------------------------------------
// Combine of split items: the parts of an item sit in consecutive partial slots; workgroup
// (slot, chunk) works if `slot` holds part 0 of its item (the others return) and covers 256
// (query, 4 dims) pairs of it: out = sum_i O_i 2^(m_i - M) / sum_i l_i 2^(m_i - M),
// M = max_i m_i (scores in log2 units). All parts' loads issue before any use.
// ---------------------------------------------------------------------------------------------
template <int HD, typename OutT>
__global__ __launch_bounds__(256) void attn_combine_kernel(const int* __restrict__ tiles, int n_whole, int n_slots,
                                                           const float* __restrict__ part, OutT* __restrict__ O,
                                                           int64_t ldo) {
  constexpr int kChunks = (kAttnBM * (HD / 4) + 255) / 256;
  const int slot = blockIdx.x / kChunks, chunk = blockIdx.x % kChunks;
  const int item = n_whole + slot;
  const int hraw = tiles[4 * item + 3];
  const int part_i = (hraw >> kAttnSplitShift) & 0xff, parts = (hraw >> kAttnPartsShift) & 0xff;
  if (part_i != 0 || parts == 0 || parts > kAttnMaxSplit || slot + parts > n_slots) return;
  const int idx = chunk * 256 + threadIdx.x;
  if (idx >= kAttnBM * (HD / 4)) return;
  const int seg_e = tiles[4 * item + 1], q0 = tiles[4 * item + 2], head = hraw & kAttnHeadMask;
  const int ql = idx / (HD / 4), d = (idx % (HD / 4)) * 4;
  if (q0 + ql >= seg_e) return;
  const int64_t slot_floats = attn_partial_floats(HD);
  const float* p0 = part + (int64_t)slot * slot_floats;
  f32x2 ml[kAttnMaxSplit];
  f32x4 o[kAttnMaxSplit];
#pragma unroll
  for (int i = 0; i < kAttnMaxSplit; ++i) {
    if (i < parts) {
      ml[i] = *reinterpret_cast<const f32x2*>(p0 + i * slot_floats + kAttnBM * HD + 2 * ql);
      o[i] = *reinterpret_cast<const f32x4*>(p0 + i * slot_floats + ql * HD + d);
    }
  }
  float M = ml[0][0];
#pragma unroll
  for (int i = 1; i < kAttnMaxSplit; ++i)
    if (i < parts) M = fmaxf(M, ml[i][0]);
  float L = 0.f;
  f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int i = 0; i < kAttnMaxSplit; ++i) {
    if (i < parts) {
      const float sc = __builtin_amdgcn_exp2f(ml[i][0] - M);
      L = fmaf(ml[i][1], sc, L);
      acc[0] = fmaf(o[i][0], sc, acc[0]); acc[1] = fmaf(o[i][1], sc, acc[1]);
      acc[2] = fmaf(o[i][2], sc, acc[2]); acc[3] = fmaf(o[i][3], sc, acc[3]);
    }
  }
  const float inv = 1.0f / L;
  if constexpr (sizeof(OutT) == 4)
    *reinterpret_cast<f32x4*>(O + (int64_t)(q0 + ql) * ldo + head * HD + d) =
        f32x4{acc[0] * inv, acc[1] * inv, acc[2] * inv, acc[3] * inv};
  else
    *reinterpret_cast<u32x2*>(O + (int64_t)(q0 + ql) * ldo + head * HD + d) =
        u32x2{pack_bf16x2(acc[0] * inv, acc[1] * inv), pack_bf16x2(acc[2] * inv, acc[3] * inv)};
}

template <int HD, typename OutT = bf16>
static int launch_combine(const int* d_tiles, int64_t n_tiles, int64_t n_whole, const float* part, OutT* out,
                          int64_t ldo, hipStream_t stream) {
  constexpr int kChunks = (kAttnBM * (HD / 4) + 255) / 256;
  const int64_t n_slots = n_tiles - n_whole;
  hipLaunchKernelGGL((attn_combine_kernel<HD, OutT>), dim3((unsigned)(n_slots * kChunks)), dim3(256), 0, stream,
                     d_tiles, (int)n_whole, (int)n_slots, part, out, ldo);
  return check_launch("attn_combine");
}

// The combine of an fp32 split list (the fp32 attention kernel writes the same partials).
int attention_combine_f32(const int* d_tiles, int64_t n_tiles, int64_t n_whole, const float* part, float* out,
                          int64_t ldo, int hd, hipStream_t stream) {
  if (hd == 64) return launch_combine<64, float>(d_tiles, n_tiles, n_whole, part, out, ldo, stream);
  if (hd == 72) return launch_combine<72, float>(d_tiles, n_tiles, n_whole, part, out, ldo, stream);
  return launch_combine<80, float>(d_tiles, n_tiles, n_whole, part, out, ldo, stream);
}

// One rotary output x*cos + rotate_half(x)*sin in the reference's bf16 arithmetic (model.py:579-582):
// x and its pair xp are bf16 values, c = (cos, sin) bf16 values; each product and the sum is
// rounded to bf16 (eager jnp ops). lower: d < hd/2, where rotate_half contributes -xp.
__device__ __forceinline__ float rope_bf16(float x, float xp, f32x2 c, bool lower) {
  const float a = round_bf16(x * c.x), b = round_bf16(xp * c.y);
  return round_bf16(lower ? a - b : a + b);
}

// Relayout for the general kernel: q/k/v [N, H*hd] (row stride ld) -> rotated, scaled Q and
// rotated K [H][Np][HDP] (dims >= hd zero), V^T [H][VROWS][Np] (rows >= hd zero, keys at vt_pos);
// token rows [N, Np) zero. Rotary pairs (d, d + hd/2) with cs[n][d] (d < hd/2).
__global__ __launch_bounds__(256) void attn_relayout_general_kernel(
    const bf16* __restrict__ q, const bf16* __restrict__ k, const bf16* __restrict__ v, int64_t ld,
    const f32x2* __restrict__ cs, int N, int Np, int hd, int HDP, int VROWS, float qscale,
    bf16* __restrict__ Qo, bf16* __restrict__ Ko, bf16* __restrict__ Vto) {
  __shared__ bf16 tv[64][129];
  const int n0 = blockIdx.x * 64, head = blockIdx.y, tid = threadIdx.x;
  const int half = hd / 2;
  for (int idx = tid; idx < 64 * HDP; idx += 256) {
    const int t = idx / HDP, d = idx % HDP, n = n0 + t;
    if (n >= Np) continue;
    float qv = 0.f, kv = 0.f;
    if (n < N && d < hd) {
      const int j = d < half ? d : d - half;
      const f32x2 c = cs[(int64_t)n * half + j];
      const int64_t base = (int64_t)n * ld + (int64_t)head * hd;
      const float a = (float)q[base + d], b = (float)k[base + d];
      const float ap = (float)q[base + (d < half ? d + half : d - half)];
      const float bp = (float)k[base + (d < half ? d + half : d - half)];
      // x*cos + rotate_half(x)*sin, rotate_half = [-x2, x1], each product and the sum rounded to
      // bf16 (model.py:579-582); q then takes the softmax pre-scale (one more rounding)
      qv = round_bf16(rope_bf16(a, ap, c, d < half)) * qscale;
      kv = rope_bf16(b, bp, c, d < half);
    }
    Qo[((int64_t)head * Np + n) * HDP + d] = (bf16)qv;
    Ko[((int64_t)head * Np + n) * HDP + d] = (bf16)kv;
  }
  for (int idx = tid; idx < 64 * VROWS; idx += 256) {
    const int t = idx / VROWS, d = idx % VROWS, n = n0 + t;
    tv[t][d] = (n < N && d < hd) ? v[(int64_t)n * ld + (int64_t)head * hd + d] : (bf16)0.f;
  }
  __syncthreads();
  for (int idx = tid; idx < 64 * VROWS; idx += 256) {
    const int d = idx / 64, t = idx % 64, n = n0 + t;
    if (n < Np) Vto[((int64_t)head * VROWS + d) * Np + vt_pos(n)] = tv[t][d];
  }
}

int attention_general(const bf16* Qb, const bf16* Kb, const bf16* Vtb, const int* d_tiles, int64_t n_tiles, int Np,
                      int H, int hd, bf16* out, int64_t ldo, hipStream_t stream, int64_t n_whole, float* part) {
  if (n_tiles == 0) return QVL_OK;
  if (hd != 72 && hd != 80)
    return set_error(QVL_ERR_UNSUPPORTED, "attention: head_dim=%d (general kernel: 72, 80)", hd);
  if (n_whole < 0) n_whole = n_tiles;
  if (hd == 72)
    hipLaunchKernelGGL(attn_fwd_qk88_kernel<72>, dim3((unsigned)n_tiles), dim3(256), 0, stream, Qb, Kb, Vtb, d_tiles,
                       Np, H, out, ldo, (int)n_whole, part);
  else
    hipLaunchKernelGGL(attn_fwd_qk88_kernel<80>, dim3((unsigned)n_tiles), dim3(256), 0, stream, Qb, Kb, Vtb, d_tiles,
                       Np, H, out, ldo, (int)n_whole, part);
  int rc = check_launch("attn_fwd_qk88");
  if (rc || n_whole >= n_tiles || !part) return rc;
  return hd == 72 ? launch_combine<72>(d_tiles, n_tiles, n_whole, part, out, ldo, stream)
                  : launch_combine<80>(d_tiles, n_tiles, n_whole, part, out, ldo, stream);
}

int attention_relayout_general(const bf16* q, const bf16* k, const bf16* v, int64_t ld, const f32x2* cs, int N, int Np,
                               int H, int hd, int HDP, int VROWS, float qscale, bf16* Qo, bf16* Ko, bf16* Vto,
                               hipStream_t stream) {
  if (VROWS > 128) return set_error(QVL_ERR_UNSUPPORTED, "relayout: head_dim too large");
  hipLaunchKernelGGL(attn_relayout_general_kernel, dim3((unsigned)(Np / 64), (unsigned)H), dim3(256), 0, stream,
                     q, k, v, ld, cs, N, Np, hd, HDP, VROWS, qscale, Qo, Ko, Vto);
  return check_launch("attn_relayout_general");
}

// Relayout for the standalone attention entry: q/k/v [N, H*hd] (row stride ld) -> rotated,
// scaled Q / rotated K [H][Np][64] and V^T [H][64][Np] (keys at vt_pos); rows [N, Np) zero-filled.
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
      q1 = round_bf16(rope_bf16(a1, a2, c, true)) * qscale;
      q2 = round_bf16(rope_bf16(a2, a1, c, false)) * qscale;
      k1 = rope_bf16(b1, b2, c, true);
      k2 = rope_bf16(b2, b1, c, false);
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
    if (n < Np) Vto[((int64_t)head * kHD + d) * Np + vt_pos(n)] = tv[t][d];
  }
}

// Key groups of the head_dim-64 kernel (thread-local override, qvl_set_attention_plan): 0 lets the
// rule decide: two groups of 4 waves per item where the items number at most 2x the CUs, so every
// item starts at once either way (two 8-wave workgroups per CU against four of 4 waves). Alone on
// MI355X, 16 heads: one 784-token image 11.8 against 12.1 us, one of 1024 tokens 13.2 against 14.3.
// Past that, part of the items wait for a slot: six 1024-token images (768 items) 36.1 against
// 32.5 us, config 3's 1024 items 49.3 against 41.6, config 2's 2304 items 166 against 160 (config
// 1's 576 uneven items were the exception, 42.5 against 43.7).
static thread_local int t_key_groups = 0;

int attention_set_plan(int key_groups) {
  if (key_groups < 0 || key_groups > 2)
    return set_error(QVL_ERR_INVALID_ARG, "attention plan: key_groups=%d (0, 1 or 2)", key_groups);
  t_key_groups = key_groups;
  return QVL_OK;
}

static int attention_key_groups(int64_t n_items) {
  if (t_key_groups) return t_key_groups;
  return n_items <= 2 * (int64_t)gemm_device_cus() ? 2 : 1;
}

int attention_hd64(const bf16* Qb, const bf16* Kb, const bf16* Vtb, const int* d_tiles, int64_t n_tiles,
                   int Np, int H, bf16* out, int64_t ldo, hipStream_t stream, int64_t n_whole, float* part) {
  if (n_tiles == 0) return QVL_OK;
  if (n_whole < 0) n_whole = n_tiles;
  if (attention_key_groups(n_tiles) == 2)
    hipLaunchKernelGGL(attn_fwd_hd64_kernel<2>, dim3((unsigned)n_tiles), dim3(512), 0, stream,
                       Qb, Kb, Vtb, d_tiles, Np, H, out, ldo, (int)n_whole, part);
  else
    hipLaunchKernelGGL(attn_fwd_hd64_kernel<1>, dim3((unsigned)n_tiles), dim3(256), 0, stream,
                       Qb, Kb, Vtb, d_tiles, Np, H, out, ldo, (int)n_whole, part);
  int rc = check_launch("attn_fwd_hd64");
  if (rc || n_whole >= n_tiles || !part) return rc;
  return launch_combine<kHD>(d_tiles, n_tiles, n_whole, part, out, ldo, stream);
}

// attn_relayout_hd64_kernel with 16-byte accesses: thread = (token t, dims [j0, j0+8) and
// [j0+32, j0+40)), 4 threads per token; the same per-element arithmetic (bit-identical output).
// V is transposed through LDS (written at the token's vt_pos column) and leaves as 16-byte rows.
// Requires q, k, v, cs 16-byte aligned and ld % 8 == 0.
__global__ __launch_bounds__(256) void attn_relayout_hd64_vec_kernel(
    const bf16* __restrict__ q, const bf16* __restrict__ k, const bf16* __restrict__ v, int64_t ld,
    const f32x2* __restrict__ cs, int N, int Np, float qscale,
    bf16* __restrict__ Qo, bf16* __restrict__ Ko, bf16* __restrict__ Vto) {
  __shared__ __attribute__((aligned(16))) bf16 tv[kHD][64 + 8];   // [dim][key position]
  const int n0 = blockIdx.x * 64, head = blockIdx.y, tid = threadIdx.x;
  const int t = tid >> 2, j0 = (tid & 3) * 8, n = n0 + t;
  const int64_t base = (int64_t)n * ld + head * kHD;
  bf16x8 qlo = {}, qhi = {}, klo = {}, khi = {}, vlo = {}, vhi = {};
  if (n < N) {
    const bf16x8 alo = *reinterpret_cast<const bf16x8*>(q + base + j0);
    const bf16x8 ahi = *reinterpret_cast<const bf16x8*>(q + base + j0 + 32);
    const bf16x8 blo = *reinterpret_cast<const bf16x8*>(k + base + j0);
    const bf16x8 bhi = *reinterpret_cast<const bf16x8*>(k + base + j0 + 32);
    vlo = *reinterpret_cast<const bf16x8*>(v + base + j0);
    vhi = *reinterpret_cast<const bf16x8*>(v + base + j0 + 32);
    f32x2 c[8];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const f32x4 w = *reinterpret_cast<const f32x4*>(cs + (int64_t)n * 32 + j0 + 2 * i);
      c[2 * i] = f32x2{w[0], w[1]};
      c[2 * i + 1] = f32x2{w[2], w[3]};
    }
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const float a1 = (float)alo[e], a2 = (float)ahi[e], b1 = (float)blo[e], b2 = (float)bhi[e];
      qlo[e] = (bf16)(round_bf16(rope_bf16(a1, a2, c[e], true)) * qscale);
      qhi[e] = (bf16)(round_bf16(rope_bf16(a2, a1, c[e], false)) * qscale);
      klo[e] = (bf16)rope_bf16(b1, b2, c[e], true);
      khi[e] = (bf16)rope_bf16(b2, b1, c[e], false);
    }
  }
  bf16* qd = Qo + ((int64_t)head * Np + n) * kHD;
  bf16* kd = Ko + ((int64_t)head * Np + n) * kHD;
  *reinterpret_cast<bf16x8*>(qd + j0) = qlo;
  *reinterpret_cast<bf16x8*>(qd + j0 + 32) = qhi;
  *reinterpret_cast<bf16x8*>(kd + j0) = klo;
  *reinterpret_cast<bf16x8*>(kd + j0 + 32) = khi;
  const int p = vt_pos(t);   // n0 is a multiple of 64: vt_pos(n0 + t) = n0 + vt_pos(t)
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    tv[j0 + e][p] = vlo[e];
    tv[j0 + 32 + e][p] = vhi[e];
  }
  __syncthreads();
#pragma unroll
  for (int i = tid; i < kHD * 8; i += 256) {
    const int d = i >> 3, c8 = (i & 7) * 8;
    *reinterpret_cast<bf16x8*>(Vto + ((int64_t)head * kHD + d) * Np + n0 + c8) =
        *reinterpret_cast<const bf16x8*>(&tv[d][c8]);
  }
}

int attention_relayout_hd64(const bf16* q, const bf16* k, const bf16* v, int64_t ld, const f32x2* cs, int N,
                            int Np, int H, float qscale, bf16* Qo, bf16* Ko, bf16* Vto, hipStream_t stream) {
  if (Np % 64) return set_error(QVL_ERR_INVALID_ARG, "relayout: Np=%d not a multiple of 64", Np);
  const auto a16 = [](const void* p) { return ((uintptr_t)p & 15) == 0; };
  const bool vec = a16(q) && a16(k) && a16(v) && a16(cs) && ld % 8 == 0 && a16(Qo) && a16(Ko) && a16(Vto);
  hipLaunchKernelGGL(vec ? attn_relayout_hd64_vec_kernel : attn_relayout_hd64_kernel,
                     dim3((unsigned)(Np / 64), (unsigned)H), dim3(256), 0, stream,
                     q, k, v, ld, cs, N, Np, qscale, Qo, Ko, Vto);
  return check_launch("attn_relayout_hd64");
}

}  // namespace qvl
