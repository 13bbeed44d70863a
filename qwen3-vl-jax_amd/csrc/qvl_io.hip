// The steps either side of encode_vision: on-device patchify of uint8 frames (the array
// preprocess_image builds after PIL's convert/resize, sample.py:86-121) and the decoder-side
// injection of vision rows into the hidden states plus the deepstack adds (model.py:874-886,
// 927-938). All are HBM-bound byte / row movement; each kernel reads its inputs once and writes
// every output element once, with 8- or 16-byte row-contiguous stores.
#include <type_traits>

#include "qvl_kernels.h"

namespace qvl {

// ---------------------------------------------------------------------------------------------
// Patchify (sample.py:86-121): value = ((u8 / 255) - 0.5) / 0.5 in fp32 (numpy's float32 ops,
// sample.py:86-87), frames padded to a multiple of Tp by repeating the last one (sample.py:93-98),
// rows in merge-block order (t, hb, wb, mi, mj) and columns (c, tp, ph, pw) (sample.py:112-119).
// One workgroup per 2-D merge block (m*m rows); VEC consecutive columns (one pw run) per step.
// ---------------------------------------------------------------------------------------------
template <int VEC, typename OutT>
__global__ __launch_bounds__(256) void patchify_kernel(const uint8_t* __restrict__ frames, int F, int H, int W,
                                                       int cin, int P, int Tp, int m, int GH, int GW,
                                                       OutT* __restrict__ out, int64_t ldo) {
  __shared__ float lut[256];
  // The 256 possible values, each by the reference's two float32 operations (IEEE division).
  lut[threadIdx.x] = ((float)threadIdx.x / 255.0f - 0.5f) / 0.5f;
  __syncthreads();

  const int K = 3 * Tp * P * P;
  const int KV = K / VEC, rows = m * m;
  const int64_t g = blockIdx.x;                       // merge block: (t * GH + hb) * GW + wb
  const int wb = (int)(g % GW);
  const int64_t tg = g / GW;
  const int hb = (int)(tg % GH), t = (int)(tg / GH);
  for (int q = threadIdx.x; q < rows * KV; q += 256) {
    const int r = q / KV, k = (q % KV) * VEC;
    const int mi = r / m, mj = r % m;
    const int pw = k % P, ph = (k / P) % P, tp = (k / (P * P)) % Tp, c = k / (P * P * Tp);
    const int f = min(t * Tp + tp, F - 1);
    const int y = (hb * m + mi) * P + ph, x = (wb * m + mj) * P + pw;
    const uint8_t* src = frames + (((int64_t)f * H + y) * W + x) * cin + c;
    OutT* dst = out + (g * rows + r) * ldo + k;
    if constexpr (VEC == 4) {
      const float v0 = lut[src[0]], v1 = lut[src[cin]], v2 = lut[src[2 * cin]], v3 = lut[src[3 * cin]];
      if constexpr (std::is_same<OutT, float>::value) {
        *reinterpret_cast<f32x4*>(dst) = f32x4{v0, v1, v2, v3};
      } else {
        *reinterpret_cast<u32x2*>(dst) = u32x2{pack_bf16x2(v0, v1), pack_bf16x2(v2, v3)};
      }
    } else {
      *dst = (OutT)lut[src[0]];
    }
  }
}

// The reference's configuration (patch 16, temporal patch 2, merge 2), with the index arithmetic
// in shifts: thread (mi, mj, ph, j) of a merge block reads the 4 pixels x CIN channels of one
// patch row quarter (x = 4j..4j+3) once per temporal slot (once when both slots repeat the same
// frame) and writes the 3 channel runs of 4 columns; a wave writes 1 KB contiguous per (c, tp).
template <int CIN, typename OutT>
__global__ __launch_bounds__(256) void patchify_p16_kernel(const uint8_t* __restrict__ frames, int F, int H, int W,
                                                           int GH, int GW, OutT* __restrict__ out, int64_t ldo) {
  constexpr int P = 16, TP = 2, M = 2;
  __shared__ float lut[256];
  lut[threadIdx.x] = ((float)threadIdx.x / 255.0f - 0.5f) / 0.5f;
  __syncthreads();
  const int64_t g = blockIdx.x;                       // merge block: (t * GH + hb) * GW + wb
  const int wb = (int)(g % GW);
  const int64_t tg = g / GW;
  const int hb = (int)(tg % GH), t = (int)(tg / GH);
  const int r = threadIdx.x >> 6, ph = (threadIdx.x >> 2) & 15, j = threadIdx.x & 3;
  const int mi = r >> 1, mj = r & 1;
  const int y = (hb * M + mi) * P + ph, x = (wb * M + mj) * P + 4 * j;
  OutT* dst = out + (g * (M * M) + r) * ldo + ph * P + 4 * j;
  uint8_t px[4 * CIN];
  int loaded = -1;
#pragma unroll
  for (int tp = 0; tp < TP; ++tp) {
    const int f = min(t * TP + tp, F - 1);
    if (f != loaded) {
      const uint8_t* src = frames + (((int64_t)f * H + y) * W + x) * CIN;
      if constexpr (CIN == 4) {
        *reinterpret_cast<u32x4*>(px) = *reinterpret_cast<const u32x4*>(src);
      } else {
        const uint32_t* s4 = reinterpret_cast<const uint32_t*>(src);
        uint32_t w3[3] = {s4[0], s4[1], s4[2]};
        __builtin_memcpy(px, w3, 12);
      }
      loaded = f;
    }
#pragma unroll
    for (int c = 0; c < 3; ++c) {
      const float v0 = lut[px[c]], v1 = lut[px[CIN + c]], v2 = lut[px[2 * CIN + c]], v3 = lut[px[3 * CIN + c]];
      OutT* d = dst + (c * TP + tp) * P * P;
      if constexpr (std::is_same<OutT, float>::value) {
        *reinterpret_cast<f32x4*>(d) = f32x4{v0, v1, v2, v3};
      } else {
        *reinterpret_cast<u32x2*>(d) = u32x2{pack_bf16x2(v0, v1), pack_bf16x2(v2, v3)};
      }
    }
  }
}

// ---------------------------------------------------------------------------------------------
// Vision-token positions (model.py:927-931 / 880-882): for each batch row, the first n_rows
// token indices s with tokens[s] == match, in increasing order, then -1 fill; count = number of
// matches (may exceed n_rows). One 1024-thread workgroup per batch row: ballot + per-wave
// popcount prefix over 1024-token chunks.
// ---------------------------------------------------------------------------------------------
__global__ __launch_bounds__(1024) void vision_positions_kernel(const int32_t* __restrict__ tokens, int64_t S,
                                                                int32_t match, int64_t n_rows,
                                                                int32_t* __restrict__ pos, int32_t* __restrict__ count) {
  __shared__ int wave_hits[16];
  const int b = blockIdx.x;
  const int32_t* tk = tokens + (int64_t)b * S;
  int32_t* pb = pos + (int64_t)b * n_rows;
  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
  int64_t base = 0;
  for (int64_t s0 = 0; s0 < S; s0 += 1024) {
    const int64_t s = s0 + threadIdx.x;
    const bool hit = s < S && tk[s] == match;
    const uint64_t bal = __ballot(hit);
    if (lane == 0) wave_hits[wv] = __popcll(bal);
    __syncthreads();
    int before = 0, total = 0;
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const int h = wave_hits[i];
      before += i < wv ? h : 0;
      total += h;
    }
    const int64_t rank = base + before + __popcll(bal & ((1ull << lane) - 1ull));
    if (hit && rank < n_rows) pb[rank] = (int32_t)s;
    base += total;
    __syncthreads();
  }
  for (int64_t r = base + threadIdx.x; r < n_rows; r += 1024) pb[r] = -1;
  if (threadIdx.x == 0) count[b] = (int32_t)base;
}

// ---------------------------------------------------------------------------------------------
// Row scatter (model.py:880-886 `_add`, 932-935 `_inject`): hidden[b, pos[b, j], :] =
// cast(rows[b, j, :]) (SET) or hidden + cast(rows) rounded to the hidden dtype (ADD), for
// pos >= 0. The reference scatters all n_rows updates, sending the unfilled ones (count <
// n_rows) to row 0 with "keep" / "+0" updates; applied in update order (XLA's CPU scatter)
// those leave hidden[b, 0] as it was before a SET, and add +0 to it after an ADD. Workgroup
// (j, b) moves one row; workgroup (n_rows, b) applies the trailing "+0" to row 0 when no
// filled entry targets it.
// ---------------------------------------------------------------------------------------------
template <typename T> __device__ __forceinline__ float ld_f(const T* p) { return (float)*p; }
template <typename T> __device__ __forceinline__ T from_f(float v) { return (T)v; }

template <int MODE, typename HT, typename RT>
__global__ __launch_bounds__(256) void scatter_rows_kernel(HT* __restrict__ hidden, int64_t S, int64_t D,
                                                           const RT* __restrict__ rows, int64_t rows_bstride,
                                                           int64_t n_rows, const int32_t* __restrict__ pos,
                                                           const int32_t* __restrict__ count) {
  const int64_t j = blockIdx.x;
  const int b = blockIdx.y;
  const int64_t cnt = count[b];
  const bool unfilled = cnt < n_rows;
  HT* hb = hidden + (int64_t)b * S * D;
  if (j == n_rows) {
    // trailing "+0" updates of the unfilled entries on row 0 (only if no filled entry is row 0)
    if (MODE == QVL_SCATTER_ADD && unfilled && pos[(int64_t)b * n_rows] != 0)
      for (int64_t d = threadIdx.x; d < D; d += 256) hb[d] = from_f<HT>(ld_f(hb + d) + 0.0f);
    return;
  }
  const int p = pos[(int64_t)b * n_rows + j];
  if (p < 0 || p >= S) return;                             // out of range: dropped, as XLA drops it
  if (MODE == QVL_SCATTER_SET && p == 0 && unfilled) return;   // overwritten by the old row 0 afterwards
  HT* h = hb + (int64_t)p * D;
  const RT* r = rows + (int64_t)b * rows_bstride + j * D;
  for (int64_t d = threadIdx.x; d < D; d += 256) {
    const HT u = from_f<HT>(ld_f(r + d));                   // feat.astype(h.dtype)
    if (MODE == QVL_SCATTER_SET) {
      h[d] = u;
    } else {
      float v = ld_f(h + d) + (float)u;                     // h + u in the hidden dtype
      v = (float)from_f<HT>(v);
      if (p == 0 && unfilled) v = (float)from_f<HT>(v + 0.0f);
      h[d] = from_f<HT>(v);
    }
  }
}

// Vector loads / stores of N (4 or 8) consecutive elements as floats: bf16 in 8- or 16-byte
// pieces, fp32 in 16-byte pieces. Stores round to the element type.
template <int N> __device__ __forceinline__ void ld_vec(const bf16* p, float (&v)[N]) {
  static_assert(N == 4 || N == 8, "ld_vec");
  if constexpr (N == 8) {
    const u32x4 w = *reinterpret_cast<const u32x4*>(p);
    v[0] = bf16_lo(w.x); v[1] = bf16_hi(w.x); v[2] = bf16_lo(w.y); v[3] = bf16_hi(w.y);
    v[4] = bf16_lo(w.z); v[5] = bf16_hi(w.z); v[6] = bf16_lo(w.w); v[7] = bf16_hi(w.w);
  } else {
    const u32x2 w = *reinterpret_cast<const u32x2*>(p);
    v[0] = bf16_lo(w.x); v[1] = bf16_hi(w.x); v[2] = bf16_lo(w.y); v[3] = bf16_hi(w.y);
  }
}
template <int N> __device__ __forceinline__ void ld_vec(const float* p, float (&v)[N]) {
#pragma unroll
  for (int i = 0; i < N; i += 4) {
    const f32x4 w = *reinterpret_cast<const f32x4*>(p + i);
    v[i] = w[0]; v[i + 1] = w[1]; v[i + 2] = w[2]; v[i + 3] = w[3];
  }
}
template <int N> __device__ __forceinline__ void st_vec(bf16* p, const float (&v)[N]) {
  static_assert(N == 4 || N == 8, "st_vec");
  if constexpr (N == 8)
    *reinterpret_cast<u32x4*>(p) = u32x4{pack_bf16x2(v[0], v[1]), pack_bf16x2(v[2], v[3]), pack_bf16x2(v[4], v[5]),
                                         pack_bf16x2(v[6], v[7])};
  else
    *reinterpret_cast<u32x2*>(p) = u32x2{pack_bf16x2(v[0], v[1]), pack_bf16x2(v[2], v[3])};
}
template <int N> __device__ __forceinline__ void st_vec(float* p, const float (&v)[N]) {
#pragma unroll
  for (int i = 0; i < N; i += 4) *reinterpret_cast<f32x4*>(p + i) = f32x4{v[i], v[i + 1], v[i + 2], v[i + 3]};
}
template <typename T> __device__ __forceinline__ float round_to(float v) {
  if constexpr (std::is_same<T, bf16>::value) return round_bf16(v);
  else return v;
}

// Same scatter, one wave per row and 16 bytes of hidden per lane step (CH elements: 8 bf16 or 4
// fp32), for rows of a multiple of 8 elements on 16-byte aligned rows; work item n_rows of each
// batch row is the trailing "+0" on row 0. Same roundings as scatter_rows_kernel.
template <int MODE, typename HT, typename RT>
__global__ __launch_bounds__(256) void scatter_rows_vec_kernel(HT* __restrict__ hidden, int64_t S, int64_t D,
                                                               const RT* __restrict__ rows, int64_t rows_bstride,
                                                               int64_t n_rows, const int32_t* __restrict__ pos,
                                                               const int32_t* __restrict__ count) {
  constexpr int CH = 16 / sizeof(HT);
  const int64_t j = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  const int b = blockIdx.y;
  if (j > n_rows) return;
  const int64_t cnt = count[b];
  const bool unfilled = cnt < n_rows;
  HT* hb = hidden + (int64_t)b * S * D;
  if (j == n_rows) {
    if (MODE == QVL_SCATTER_ADD && unfilled && pos[(int64_t)b * n_rows] != 0)
      for (int64_t d = (int64_t)lane * CH; d < D; d += 64 * CH) {
        float h[CH];
        ld_vec<CH>(hb + d, h);
#pragma unroll
        for (int e = 0; e < CH; ++e) h[e] += 0.0f;
        st_vec<CH>(hb + d, h);
      }
    return;
  }
  const int p = pos[(int64_t)b * n_rows + j];
  if (p < 0 || p >= S) return;                             // out of range: dropped, as XLA drops it
  if (MODE == QVL_SCATTER_SET && p == 0 && unfilled) return;   // overwritten by the old row 0 afterwards
  HT* h = hb + (int64_t)p * D;
  const RT* r = rows + (int64_t)b * rows_bstride + j * D;
  for (int64_t d = (int64_t)lane * CH; d < D; d += 64 * CH) {
    float u[CH];
    ld_vec<CH>(r + d, u);
#pragma unroll
    for (int e = 0; e < CH; ++e) u[e] = round_to<HT>(u[e]);        // feat.astype(h.dtype)
    if (MODE == QVL_SCATTER_ADD) {
      float hv[CH];
      ld_vec<CH>(h + d, hv);
#pragma unroll
      for (int e = 0; e < CH; ++e) {
        float v = round_to<HT>(hv[e] + u[e]);                      // h + u in the hidden dtype
        if (p == 0 && unfilled) v = round_to<HT>(v + 0.0f);
        u[e] = v;
      }
    }
    st_vec<CH>(h + d, u);
  }
}

// ---------------------------------------------------------------------------------------------
// Row gather (model.py:809-812 shuffle / 845-848 unshuffle of the window path): out row r is
// in row idx[r / group] * group + r % group (row r itself without idx), cast to the output dtype;
// out columns [width, pad_to) are written zero (the tower's bf16 pixel rows padded to a multiple
// of 64 for the patch-embed GEMM). VEC elements per step.
// ---------------------------------------------------------------------------------------------
template <int VEC, typename IT, typename OT>
__global__ __launch_bounds__(256) void gather_rows_kernel(const IT* __restrict__ src, int64_t ld_src,
                                                          OT* __restrict__ dst, int64_t ld_dst,
                                                          const int32_t* __restrict__ idx, int group, int64_t width,
                                                          int64_t pad_to) {
  const int64_t r = blockIdx.x;
  const int64_t sr = idx ? (int64_t)idx[r / group] * group + r % group : r;
  const IT* s = src + sr * ld_src;
  OT* d = dst + r * ld_dst;
  for (int64_t c = (int64_t)threadIdx.x * VEC; c < width; c += 256 * VEC) {
    if constexpr (VEC == 4 && std::is_same<IT, float>::value) {
      const f32x4 v = *reinterpret_cast<const f32x4*>(s + c);
      if constexpr (std::is_same<OT, float>::value) *reinterpret_cast<f32x4*>(d + c) = v;
      else *reinterpret_cast<u32x2*>(d + c) = u32x2{pack_bf16x2(v[0], v[1]), pack_bf16x2(v[2], v[3])};
    } else if constexpr (VEC == 4) {
      const u32x2 v = *reinterpret_cast<const u32x2*>(s + c);
      if constexpr (std::is_same<OT, float>::value)
        *reinterpret_cast<f32x4*>(d + c) = f32x4{bf16_lo(v.x), bf16_hi(v.x), bf16_lo(v.y), bf16_hi(v.y)};
      else *reinterpret_cast<u32x2*>(d + c) = v;
    } else {
      d[c] = (OT)(float)s[c];
    }
  }
  for (int64_t c = width + threadIdx.x; c < pad_to; c += 256) d[c] = (OT)0.f;
}

int gather_rows_pad(void* stream, int32_t src_dtype, const void* src, int64_t ld_src, int32_t dst_dtype,
                         void* dst, int64_t ld_dst, const int32_t* idx, int64_t n_rows, int32_t group, int64_t width,
                         int64_t pad_to) {
  const bool sok = src_dtype == QVL_DTYPE_F32 || src_dtype == QVL_DTYPE_BF16;
  const bool dok = dst_dtype == QVL_DTYPE_F32 || dst_dtype == QVL_DTYPE_BF16;
  if (!sok || !dok) return set_error(QVL_ERR_UNSUPPORTED, "gather_rows: dtypes %d/%d", src_dtype, dst_dtype);
  if (n_rows < 0 || width < 0 || group <= 0 || n_rows % group || ld_src < width || pad_to < width || ld_dst < pad_to)
    return set_error(QVL_ERR_INVALID_ARG, "gather_rows: bad sizes");
  if (n_rows == 0 || pad_to == 0) return QVL_OK;
  if (n_rows > 0x7fffffffLL) return set_error(QVL_ERR_UNSUPPORTED, "gather_rows: n_rows");
  if (!src || !dst) return set_error(QVL_ERR_INVALID_ARG, "gather_rows: NULL pointer");
  const size_t sa = src_dtype == QVL_DTYPE_F32 ? 16 : 8, da = dst_dtype == QVL_DTYPE_F32 ? 16 : 8;
  const bool vec = width % 4 == 0 && ld_src % 4 == 0 && ld_dst % 4 == 0 && (uintptr_t)src % sa == 0 &&
                   (uintptr_t)dst % da == 0;
  hipStream_t st = (hipStream_t)stream;
  const dim3 grid((unsigned)n_rows);
#define QVL_GATHER(V, IT, OT)                                                                                 \
  hipLaunchKernelGGL((gather_rows_kernel<V, IT, OT>), grid, dim3(256), 0, st, (const IT*)src, ld_src, (OT*)dst, \
                     ld_dst, idx, group, width, pad_to)
  const bool sb = src_dtype == QVL_DTYPE_BF16, db = dst_dtype == QVL_DTYPE_BF16;
  if (vec) {
    if (sb && db) QVL_GATHER(4, bf16, bf16); else if (sb) QVL_GATHER(4, bf16, float);
    else if (db) QVL_GATHER(4, float, bf16); else QVL_GATHER(4, float, float);
  } else {
    if (sb && db) QVL_GATHER(1, bf16, bf16); else if (sb) QVL_GATHER(1, bf16, float);
    else if (db) QVL_GATHER(1, float, bf16); else QVL_GATHER(1, float, float);
  }
#undef QVL_GATHER
  return check_launch("gather_rows");
}

}  // namespace qvl

using namespace qvl;

extern "C" {

int qvl_patchify(void* stream, int32_t dtype, const uint8_t* frames, int64_t n_frames, int64_t height, int64_t width,
                 int32_t channels, int32_t patch_size, int32_t temporal_patch_size, int32_t merge_size, void* out,
                 int64_t ld_out) {
  if (dtype != QVL_DTYPE_F32 && dtype != QVL_DTYPE_BF16) return set_error(QVL_ERR_UNSUPPORTED, "patchify: dtype %d", dtype);
  if (n_frames <= 0 || height <= 0 || width <= 0 || (channels != 3 && channels != 4) || patch_size <= 0 ||
      temporal_patch_size <= 0 || merge_size <= 0)
    return set_error(QVL_ERR_INVALID_ARG, "patchify: bad sizes");
  if (height % patch_size || width % patch_size)
    return set_error(QVL_ERR_INVALID_ARG, "patchify: dimensions must be divisible by patch_size");
  const int64_t gh = height / patch_size, gw = width / patch_size;
  if (gh % merge_size || gw % merge_size)
    return set_error(QVL_ERR_INVALID_ARG, "patchify: grid must be divisible by spatial_merge_size");
  const int64_t K = 3LL * temporal_patch_size * patch_size * patch_size;
  if (ld_out < K) return set_error(QVL_ERR_INVALID_ARG, "patchify: ld_out %lld < %lld", (long long)ld_out, (long long)K);
  if (!frames || !out) return set_error(QVL_ERR_INVALID_ARG, "patchify: NULL pointer");
  if (K * merge_size * merge_size > (1LL << 30) || height * width * channels * n_frames > (1LL << 40))
    return set_error(QVL_ERR_UNSUPPORTED, "patchify: sizes");
  const int64_t gt = (n_frames + temporal_patch_size - 1) / temporal_patch_size;
  const int64_t blocks = gt * (gh / merge_size) * (gw / merge_size);
  if (blocks == 0) return QVL_OK;
  if (blocks > 0x7fffffffLL) return set_error(QVL_ERR_UNSUPPORTED, "patchify: too many merge blocks");
  const bool vec = patch_size % 4 == 0 && ld_out % 4 == 0 &&
                   ((uintptr_t)out % (dtype == QVL_DTYPE_F32 ? 16 : 8)) == 0;
  hipStream_t st = (hipStream_t)stream;
  const int F = (int)n_frames, H = (int)height, W = (int)width, P = patch_size, Tp = temporal_patch_size,
            m = merge_size, GH = (int)(gh / merge_size), GW = (int)(gw / merge_size);
  const dim3 grid((unsigned)blocks);
  const bool p16 = vec && P == 16 && Tp == 2 && m == 2 && (uintptr_t)frames % 4 == 0;
  if (p16) {
    if (dtype == QVL_DTYPE_F32) {
      if (channels == 3) hipLaunchKernelGGL((patchify_p16_kernel<3, float>), grid, dim3(256), 0, st, frames, F, H, W, GH, GW, (float*)out, ld_out);
      else hipLaunchKernelGGL((patchify_p16_kernel<4, float>), grid, dim3(256), 0, st, frames, F, H, W, GH, GW, (float*)out, ld_out);
    } else {
      if (channels == 3) hipLaunchKernelGGL((patchify_p16_kernel<3, bf16>), grid, dim3(256), 0, st, frames, F, H, W, GH, GW, (bf16*)out, ld_out);
      else hipLaunchKernelGGL((patchify_p16_kernel<4, bf16>), grid, dim3(256), 0, st, frames, F, H, W, GH, GW, (bf16*)out, ld_out);
    }
    return check_launch("patchify");
  }
  if (dtype == QVL_DTYPE_F32) {
    if (vec) hipLaunchKernelGGL((patchify_kernel<4, float>), grid, dim3(256), 0, st, frames, F, H, W, channels, P, Tp, m, GH, GW, (float*)out, ld_out);
    else hipLaunchKernelGGL((patchify_kernel<1, float>), grid, dim3(256), 0, st, frames, F, H, W, channels, P, Tp, m, GH, GW, (float*)out, ld_out);
  } else {
    if (vec) hipLaunchKernelGGL((patchify_kernel<4, bf16>), grid, dim3(256), 0, st, frames, F, H, W, channels, P, Tp, m, GH, GW, (bf16*)out, ld_out);
    else hipLaunchKernelGGL((patchify_kernel<1, bf16>), grid, dim3(256), 0, st, frames, F, H, W, channels, P, Tp, m, GH, GW, (bf16*)out, ld_out);
  }
  return check_launch("patchify");
}

int qvl_gather_rows(void* stream, int32_t src_dtype, const void* src, int64_t ld_src, int32_t dst_dtype, void* dst,
                    int64_t ld_dst, const int32_t* idx, int64_t n_rows, int32_t group, int64_t width) {
  if (!idx && n_rows > 0 && width > 0) return set_error(QVL_ERR_INVALID_ARG, "gather_rows: NULL pointer");
  return gather_rows_pad(stream, src_dtype, src, ld_src, dst_dtype, dst, ld_dst, idx, n_rows, group, width, width);
}


int qvl_vision_positions(void* stream, const int32_t* tokens, int64_t batch, int64_t seq_len, int32_t match,
                         int64_t n_rows, int32_t* pos, int32_t* count) {
  if (batch < 0 || seq_len < 0 || n_rows < 0) return set_error(QVL_ERR_INVALID_ARG, "vision_positions: bad sizes");
  if (seq_len > 0x7fffffffLL || batch > 0x7fffffffLL) return set_error(QVL_ERR_UNSUPPORTED, "vision_positions: sizes");
  if (batch == 0) return QVL_OK;
  if ((!tokens && seq_len > 0) || (!pos && n_rows > 0) || !count)
    return set_error(QVL_ERR_INVALID_ARG, "vision_positions: NULL pointer");
  hipLaunchKernelGGL(vision_positions_kernel, dim3((unsigned)batch), dim3(1024), 0, (hipStream_t)stream, tokens, seq_len,
                     match, n_rows, pos, count);
  return check_launch("vision_positions");
}

int qvl_scatter_vision_rows(void* stream, int32_t mode, int32_t hidden_dtype, void* hidden, int64_t batch,
                            int64_t seq_len, int64_t dim, int32_t rows_dtype, const void* rows,
                            int64_t rows_batch_stride, int64_t n_rows, const int32_t* pos, const int32_t* count) {
  if (mode != QVL_SCATTER_SET && mode != QVL_SCATTER_ADD) return set_error(QVL_ERR_INVALID_ARG, "scatter_vision_rows: mode %d", mode);
  const bool hok = hidden_dtype == QVL_DTYPE_F32 || hidden_dtype == QVL_DTYPE_BF16;
  const bool rok = rows_dtype == QVL_DTYPE_F32 || rows_dtype == QVL_DTYPE_BF16;
  if (!hok || !rok) return set_error(QVL_ERR_UNSUPPORTED, "scatter_vision_rows: dtypes %d/%d", hidden_dtype, rows_dtype);
  if (batch < 0 || seq_len < 0 || dim < 0 || n_rows < 0 || rows_batch_stride < 0)
    return set_error(QVL_ERR_INVALID_ARG, "scatter_vision_rows: bad sizes");
  if (batch == 0 || n_rows == 0 || dim == 0) return QVL_OK;
  if (batch > 65535 || n_rows >= 0x7fffffffLL) return set_error(QVL_ERR_UNSUPPORTED, "scatter_vision_rows: sizes");
  if (!hidden || !rows || !pos || !count) return set_error(QVL_ERR_INVALID_ARG, "scatter_vision_rows: NULL pointer");
  hipStream_t st = (hipStream_t)stream;
  const int64_t rb_bytes = rows_dtype == QVL_DTYPE_BF16 ? 2 : 4;
  const bool vec = dim % 8 == 0 && (uintptr_t)hidden % 16 == 0 && (uintptr_t)rows % 16 == 0 &&
                   (rows_batch_stride * rb_bytes) % 16 == 0;
  const dim3 grid(vec ? (unsigned)((n_rows + 1 + 3) / 4) : (unsigned)(n_rows + 1), (unsigned)batch);
#define QVL_SCATTER(M, HT, RT)                                                                                 \
  do {                                                                                                          \
    if (vec) hipLaunchKernelGGL((scatter_rows_vec_kernel<M, HT, RT>), grid, dim3(256), 0, st, (HT*)hidden,     \
                                seq_len, dim, (const RT*)rows, rows_batch_stride, n_rows, pos, count);          \
    else hipLaunchKernelGGL((scatter_rows_kernel<M, HT, RT>), grid, dim3(256), 0, st, (HT*)hidden, seq_len, dim, \
                            (const RT*)rows, rows_batch_stride, n_rows, pos, count);                            \
  } while (0)
  const bool hb = hidden_dtype == QVL_DTYPE_BF16, rb = rows_dtype == QVL_DTYPE_BF16;
  if (mode == QVL_SCATTER_SET) {
    if (hb && rb) QVL_SCATTER(QVL_SCATTER_SET, bf16, bf16);
    else if (hb) QVL_SCATTER(QVL_SCATTER_SET, bf16, float);
    else if (rb) QVL_SCATTER(QVL_SCATTER_SET, float, bf16);
    else QVL_SCATTER(QVL_SCATTER_SET, float, float);
  } else {
    if (hb && rb) QVL_SCATTER(QVL_SCATTER_ADD, bf16, bf16);
    else if (hb) QVL_SCATTER(QVL_SCATTER_ADD, bf16, float);
    else if (rb) QVL_SCATTER(QVL_SCATTER_ADD, float, bf16);
    else QVL_SCATTER(QVL_SCATTER_ADD, float, float);
  }
#undef QVL_SCATTER
  return check_launch("scatter_vision_rows");
}

}  // extern "C"
