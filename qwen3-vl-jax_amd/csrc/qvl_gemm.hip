// bf16 MFMA GEMM with fused epilogues for every Dense of the vision tower.
//
//   y[M, N] = epi(x[M, K] . W[N, K]^T + bias)     (nn.Dense: model.py:556, 570, 601, 611-613, 655-656)
//
// Both operands are K-contiguous ("TN"): activations are row-major [tokens, features] and the
// packed weights are the Flax kernel transposed. One workgroup of 4 waves computes a BM x BN
// tile; each wave owns a (BM/2) x (BN/2) sub-tile built from v_mfma_f32_32x32x16_bf16 blocks.
// The MFMA "A" operand is the weight tile and "B" the activation tile, so each lane's
// accumulator holds one token row and runs of 4 consecutive output features: the epilogue
// stores 8-byte pieces of a row instead of scattered 2-byte elements.
//
// K loop: BK = 64, operands staged through LDS (XOR-swizzled 16-byte chunks, conflict-free for
// the fragment reads), double-buffered so one barrier per K step suffices; the next K step's
// global loads are in flight while the current one is multiplied.
#include "qvl_kernels.h"

namespace qvl {

constexpr int kBK = 64;

template <int BM, int BN>
struct GemmShape {
  static constexpr int TM = BM / 2, TN = BN / 2;      // wave sub-tile
  static constexpr int MB = TM / 32, NB = TN / 32;    // 32x32 MFMA blocks per wave
  static constexpr int CHUNKS = (BM + BN) * (kBK / 8);   // 16-byte chunks per K step
  static constexpr int PER_THREAD = CHUNKS / 256;
  static_assert(CHUNKS % 256 == 0, "tile must split evenly over 256 threads");
  static constexpr int LDS_ELEMS = (BM + BN) * kBK;    // one stage
};

// LDS element offset of (row, 16-byte chunk) with the XOR swizzle.
__device__ __forceinline__ int lds_off(int row, int chunk) { return row * kBK + ((chunk ^ (row & 7)) << 3); }

template <int BM, int BN, int EPI>
__global__ __launch_bounds__(256, 1) void gemm_bf16_kernel(GemmParams p) {
  using S = GemmShape<BM, BN>;
  extern __shared__ __attribute__((aligned(16))) bf16 smem[];   // [2][BM+BN][64]

  const int tiles_n = (p.N + BN - 1) / BN;
  const int tiles_m = (p.M + BM - 1) / BM;
  const int tile = xcd_remap(blockIdx.x, tiles_m * tiles_n);
  const int tm = tile / tiles_n, tn = tile % tiles_n;
  const int m0 = tm * BM, n0 = tn * BN;

  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = tid >> 6;
  const int wm = wave & 1, wn = wave >> 1;
  const int l32 = lane & 31, hh = lane >> 5;

  const __amdgpu_buffer_rsrc_t rx = make_rsrc(p.x, (uint32_t)((int64_t)p.M * p.lda * 2));
  const __amdgpu_buffer_rsrc_t rw = make_rsrc(p.w, (uint32_t)((int64_t)p.N * p.K * 2));

  // Global->register staging: chunk id c = i*256 + tid, row = c / 8, 16-byte column chunk c % 8.
  u32x4 stage[S::PER_THREAD];
  auto load_global = [&](int k0) {
#pragma unroll
    for (int i = 0; i < S::PER_THREAD; ++i) {
      const int c = i * 256 + tid;
      const int row = c >> 3, ch = c & 7;
      if (row < BM) {
        const uint32_t off = (uint32_t)(((int64_t)(m0 + row) * p.lda + k0 + ch * 8) * 2);
        stage[i] = (m0 + row < p.M) ? buf_load16(rx, off) : u32x4{0, 0, 0, 0};
      } else {
        const int r = row - BM;
        const uint32_t off = (uint32_t)(((int64_t)(n0 + r) * p.K + k0 + ch * 8) * 2);
        stage[i] = (n0 + r < p.N) ? buf_load16(rw, off) : u32x4{0, 0, 0, 0};
      }
    }
  };
  auto store_lds = [&](int buf) {
    bf16* base = smem + buf * S::LDS_ELEMS;
#pragma unroll
    for (int i = 0; i < S::PER_THREAD; ++i) {
      const int c = i * 256 + tid;
      const int row = c >> 3, ch = c & 7;
      *reinterpret_cast<u32x4*>(base + lds_off(row, ch)) = stage[i];
    }
  };

  f32x16 acc[S::NB][S::MB];
#pragma unroll
  for (int a = 0; a < S::NB; ++a)
#pragma unroll
    for (int b = 0; b < S::MB; ++b) acc[a][b] = f32x16{};

  const int KT = p.K / kBK;
  load_global(0);
  store_lds(0);
  __syncthreads();

  for (int kt = 0; kt < KT; ++kt) {
    const int cur = kt & 1;
    if (kt + 1 < KT) load_global((kt + 1) * kBK);
    const bf16* xs = smem + cur * S::LDS_ELEMS;            // rows [0, BM)
    const bf16* ws = xs + BM * kBK;                        // rows [0, BN)
#pragma unroll
    for (int ks = 0; ks < kBK / 16; ++ks) {
      const int ch = ks * 2 + hh;
      bf16x8 wf[S::NB], xf[S::MB];
#pragma unroll
      for (int a = 0; a < S::NB; ++a)
        wf[a] = *reinterpret_cast<const bf16x8*>(ws + lds_off(wn * S::TN + a * 32 + l32, ch));
#pragma unroll
      for (int b = 0; b < S::MB; ++b)
        xf[b] = *reinterpret_cast<const bf16x8*>(xs + lds_off(wm * S::TM + b * 32 + l32, ch));
#pragma unroll
      for (int a = 0; a < S::NB; ++a)
#pragma unroll
        for (int b = 0; b < S::MB; ++b)
          acc[a][b] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(wf[a], xf[b], acc[a][b], 0, 0, 0);
    }
    if (kt + 1 < KT) store_lds(cur ^ 1);
    __syncthreads();
  }

  // ---------------------------------------------------------------------------------------
  // Epilogue. Block (a, b), register r: n = nbase + 8*(r/4) + 4*hh + r%4, m = mbase + l32.
  // ---------------------------------------------------------------------------------------
  if constexpr (EPI == kEpiQkvRope) {
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
            bf16* vt = p.vt + (int64_t)head * 64 * p.Np;
#pragma unroll
            for (int e = 0; e < 4; ++e) {
              vt[(int64_t)(d + e) * p.Np + m] = (bf16)lo[e];
              vt[(int64_t)(d + e + 32) * p.Np + m] = (bf16)hi[e];
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

template <int BM, int BN, int EPI>
static int launch_gemm(const GemmParams& p, hipStream_t stream) {
  using S = GemmShape<BM, BN>;
  const int tiles = ((p.M + BM - 1) / BM) * ((p.N + BN - 1) / BN);
  const size_t lds = 2 * S::LDS_ELEMS * sizeof(bf16);
  static bool attr_set = false;   // benign race: every thread sets the same value
  if (!attr_set) {
    if (hipFuncSetAttribute((const void*)gemm_bf16_kernel<BM, BN, EPI>,
                            hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds) != hipSuccess)
      return set_error(QVL_ERR_LAUNCH, "gemm_bf16: cannot reserve %zu bytes of LDS", lds);
    attr_set = true;
  }
  hipLaunchKernelGGL((gemm_bf16_kernel<BM, BN, EPI>), dim3(tiles), dim3(256), lds, stream, p);
  return check_launch("gemm_bf16");
}

// Tile choice: big 256x256 tiles keep LDS traffic per MFMA lowest; narrower tiles are used when
// the big ones would leave most of the 256 CUs idle on the last wave of workgroups.
template <int EPI>
static int dispatch_gemm(const GemmParams& p, hipStream_t stream) {
  if constexpr (EPI == kEpiQkvRope) return launch_gemm<256, 256, EPI>(p, stream);
  const int64_t big = ((p.M + 255) / 256) * ((p.N + 255) / 256);
  if (big >= 768) return launch_gemm<256, 256, EPI>(p, stream);
  return launch_gemm<256, 128, EPI>(p, stream);
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
