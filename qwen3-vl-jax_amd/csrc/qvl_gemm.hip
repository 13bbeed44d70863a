// bf16 MFMA GEMM with fused epilogues for every Dense of the vision tower.
//
//   y[M, N] = epi(x[M, K] . W[N, K]^T + bias)     (nn.Dense: model.py:556, 570, 601, 611-613, 655-656)
//
// Both operands are K-contiguous ("TN"): activations are row-major [tokens, features] and the
// packed weights are the Flax kernel transposed. A workgroup of 8 waves (two per SIMD) computes a
// BM x BN tile; each wave owns a (BM/4) x (BN/2) sub-tile of v_mfma_f32_32x32x16_bf16 blocks.
// The MFMA "A" operand is the weight tile and "B" the activation tile, so each lane's
// accumulator holds one token row and runs of 4 consecutive output features: the epilogue
// stores 8-byte pieces of a row instead of scattered 2-byte elements.
//
// K loop (BK = 64): operands reach LDS by DMA (buffer_load ... lds, no register staging),
// double-buffered with one barrier per K step; the LDS layout is XOR-swizzled for the 16-lane,
// 64-bank fragment reads; fragments are double-buffered across the four 16-deep k-steps and
// interleaved one read per MFMA.
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
  static constexpr int ROWS_PER_PASS = THREADS / 8;     // rows one staging pass covers
  static_assert(BM % ROWS_PER_PASS == 0 && BN % ROWS_PER_PASS == 0, "staging must tile the operands");
  static constexpr int XPT = BM / ROWS_PER_PASS, WPT = BN / ROWS_PER_PASS;
  static constexpr int LDS_ELEMS = (BM + BN) * kBK;    // one stage
};

// LDS element offset of (row, 16-byte chunk). Rows are 128 bytes; the LDS serves a 16-byte read
// for 16 lanes per clock across 64 banks, i.e. two rows' worth, so rows r and r+1 fall in
// different bank halves and the chunk is XOR-swizzled with (r/2) % 8: the 16 consecutive rows a
// fragment read touches in one clock hit 16 distinct 16-byte bank groups.
__device__ __forceinline__ int lds_off(int row, int chunk) {
  return row * kBK + ((chunk ^ ((row >> 1) & 7)) << 3);
}

template <int BM, int BN, int WM, int WN, int EPI>
__global__ __launch_bounds__(64 * WM * WN, 1) void gemm_bf16_kernel(GemmParams p) {
  using S = GemmShape<BM, BN, WM, WN>;
  extern __shared__ __attribute__((aligned(16))) bf16 smem[];   // [2][BM+BN][64]

  const int tiles_n = (p.N + BN - 1) / BN;
  const int tiles_m = (p.M + BM - 1) / BM;
  const int tile = xcd_remap(blockIdx.x, tiles_m * tiles_n);
  const int tm = tile / tiles_n, tn = tile % tiles_n;
  const int m0 = tm * BM, n0 = tn * BN;

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
  auto dma_stage = [&](int k0, int stage) {
    const uint32_t xa = lds_base + stage * S::LDS_ELEMS * 2, wa = xa + BM * kBK * 2;
#pragma unroll
    for (int i = 0; i < S::XPT; ++i)
      dma16(rxw, xv, (uint32_t)((i * S::ROWS_PER_PASS * p.lda + k0) * 2), xa + (i * S::ROWS_PER_PASS + wave * 8) * kBK * 2);
#pragma unroll
    for (int i = 0; i < S::WPT; ++i)
      dma16(rww, wv, (uint32_t)((i * S::ROWS_PER_PASS * p.K + k0) * 2), wa + (i * S::ROWS_PER_PASS + wave * 8) * kBK * 2);
  };

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

  const int KT = p.K / kBK;
  dma_stage(0, 0);
  wait_dma();
  __syncthreads();
  read_frags(smem, 0, 0);

  for (int kt = 0; kt < KT; ++kt) {
    const int cur = kt & 1;
    const bf16* xs = smem + cur * S::LDS_ELEMS;
    const bool more = kt + 1 < KT;
    if (more) dma_stage((kt + 1) * kBK, cur ^ 1);
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
    wait_dma();
    __syncthreads();
    if (more) read_frags(smem + (cur ^ 1) * S::LDS_ELEMS, 0, 0);
  }

  // ---------------------------------------------------------------------------------------
  // Epilogue. Block (a, b), register r: n = nbase + 8*(r/4) + 4*hh + r%4, m = mbase + l32.
  // ---------------------------------------------------------------------------------------
  if constexpr (EPI == kEpiQkvRope) {
    static_assert(S::NB == 4, "the rotary epilogue needs 128-feature (two-head) wave tiles");
    // Wave sub-tile covers TN = 128 features = two heads of 64 (n0 + wn*TN is a multiple of
    // 128, D a multiple of 128): blocks (0,1) are head hA dims [0,32) / [32,64), (2,3) head hA+1.
    const int nw = n0 + wn * S::TN;
    if (nw >= p.N) return;
    const int which = nw / p.D;                 // 0 = q, 1 = k, 2 = v
    const int head0 = (nw % p.D) / 64;
#pragma unroll
    for (int b = 0; b < S::MB; ++b) {
      const int m = m0 + wm * S::TM + b * 32 + l32;
      if (m >= p.Np) continue;
      const bool live = m < p.M;
#pragma unroll
      for (int hp = 0; hp < S::NB / 2; ++hp) {
        const int head = head0 + hp;
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          const int d = 8 * g + 4 * hh;          // first of 4 consecutive dims in [0, 32)
          float lo[4], hi[4];
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            const int n = nw + hp * 64 + d + e;
            lo[e] = live ? acc[2 * hp][b][4 * g + e] + p.bias[n] : 0.f;
            hi[e] = live ? acc[2 * hp + 1][b][4 * g + e] + p.bias[n + 32] : 0.f;
          }
          if (which == 2) {
            bf16* vt = p.vt + (int64_t)head * 64 * p.Np + vt_pos(m);
#pragma unroll
            for (int e = 0; e < 4; ++e) {
              vt[(int64_t)(d + e) * p.Np] = (bf16)lo[e];
              vt[(int64_t)(d + e + 32) * p.Np] = (bf16)hi[e];
            }
          } else {
            float o1[4], o2[4];
            if (live) {
              const f32x2* csr = p.cs + (int64_t)m * 32 + d;
#pragma unroll
              for (int e = 0; e < 4; ++e) {
                const f32x2 t = csr[e];
                o1[e] = lo[e] * t.x - hi[e] * t.y;     // x*cos + rotate_half(x)*sin, d < 32
                o2[e] = hi[e] * t.x + lo[e] * t.y;     // d + 32
              }
            } else {
#pragma unroll
              for (int e = 0; e < 4; ++e) { o1[e] = 0.f; o2[e] = 0.f; }
            }
            const float sc = which == 0 ? p.qscale : 1.0f;
            bf16* dst = (which == 0 ? p.q : p.k) + ((int64_t)head * p.Np + m) * 64;
            u32x2 v1 = {pack_bf16x2(o1[0] * sc, o1[1] * sc), pack_bf16x2(o1[2] * sc, o1[3] * sc)};
            u32x2 v2 = {pack_bf16x2(o2[0] * sc, o2[1] * sc), pack_bf16x2(o2[2] * sc, o2[3] * sc)};
            *reinterpret_cast<u32x2*>(dst + d) = v1;
            *reinterpret_cast<u32x2*>(dst + d + 32) = v2;
          }
        }
      }
    }
  } else {
#pragma unroll
    for (int a = 0; a < S::NB; ++a) {
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const int n = n0 + wn * S::TN + a * 32 + 8 * g + 4 * hh;
        if (n >= p.N) continue;
        const f32x4 bv = *reinterpret_cast<const f32x4*>(p.bias + n);
#pragma unroll
        for (int b = 0; b < S::MB; ++b) {
          const int m = m0 + wm * S::TM + b * 32 + l32;
          if (m >= p.M) continue;
          float v[4];
#pragma unroll
          for (int e = 0; e < 4; ++e) v[e] = acc[a][b][4 * g + e] + bv[e];
          if constexpr (EPI == kEpiBiasGelu) {
#pragma unroll
            for (int e = 0; e < 4; ++e) v[e] = gelu_tanh(v[e]);
          }
          if constexpr (EPI == kEpiBiasResidual) {
            const u32x2 r = *reinterpret_cast<const u32x2*>(p.res + (int64_t)m * p.ldr + n);
            v[0] += bf16_lo(r.x); v[1] += bf16_hi(r.x); v[2] += bf16_lo(r.y); v[3] += bf16_hi(r.y);
          }
          u32x2 o = {pack_bf16x2(v[0], v[1]), pack_bf16x2(v[2], v[3])};
          *reinterpret_cast<u32x2*>(p.y + (int64_t)m * p.ldc + n) = o;
        }
      }
    }
  }
}

template <int BM, int BN, int WM, int WN, int EPI>
static int launch_gemm(const GemmParams& p, hipStream_t stream) {
  using S = GemmShape<BM, BN, WM, WN>;
  const int tiles = ((p.M + BM - 1) / BM) * ((p.N + BN - 1) / BN);
  const size_t lds = 2 * S::LDS_ELEMS * sizeof(bf16);
  static bool attr_set = false;   // benign race: every thread sets the same value
  if (!attr_set) {
    if (hipFuncSetAttribute((const void*)gemm_bf16_kernel<BM, BN, WM, WN, EPI>,
                            hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds) != hipSuccess)
      return set_error(QVL_ERR_LAUNCH, "gemm_bf16: cannot reserve %zu bytes of LDS", lds);
    attr_set = true;
  }
  hipLaunchKernelGGL((gemm_bf16_kernel<BM, BN, WM, WN, EPI>), dim3(tiles), dim3(S::THREADS), lds, stream, p);
  return check_launch("gemm_bf16");
}

// Tile choice: 256x256 tiles on 8 waves (two per SIMD, 64x128 each) keep LDS traffic per MFMA
// low while a second wave hides each wave's memory latency; 256x128 tiles (8 waves of 64x64)
// when 256x256 would leave most CUs idle on the last round of workgroups.
template <int EPI>
static int dispatch_gemm(const GemmParams& p, hipStream_t stream) {
  if constexpr (EPI == kEpiQkvRope) {
    return launch_gemm<256, 256, 4, 2, EPI>(p, stream);
  } else {
    const int64_t big = ((p.M + 255) / 256) * ((p.N + 255) / 256);
    if (big >= 768) return launch_gemm<256, 256, 4, 2, EPI>(p, stream);
    return launch_gemm<256, 128, 4, 2, EPI>(p, stream);
  }
}

int gemm_bf16(const GemmParams& p, int epi, hipStream_t stream) {
  switch (epi) {
    case kEpiBias: return dispatch_gemm<kEpiBias>(p, stream);
    case kEpiBiasGelu: return dispatch_gemm<kEpiBiasGelu>(p, stream);
    case kEpiBiasResidual: return dispatch_gemm<kEpiBiasResidual>(p, stream);
    case kEpiQkvRope: return dispatch_gemm<kEpiQkvRope>(p, stream);
  }
  return set_error(QVL_ERR_INVALID_ARG, "unknown epilogue %d", epi);
}

}  // namespace qvl
