// GPU-free host side of libqvl: error plumbing and the tower's integer metadata (bit-exact with the
// reference's numpy): grid counts, cu_seqlens, rotary ids, pos-embed taps, window index, the
// attention work lists and the rotary inverse frequencies. Plain C++ (no HIP): the CPU sanitizer
// build (tests/test_host_sanitizer.py) compiles this file on its own.
#include <math.h>
#include <stdarg.h>
#include <stdio.h>
#include <string.h>

#include <algorithm>
#include <array>
#include <vector>

#include "qvl_host_common.h"

namespace qvl {

static thread_local char g_err[512];

int set_error(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof(g_err), fmt, ap);
  va_end(ap);
  return code;
}

// Float32 value of bf16(x) with round-to-nearest-even (host).
static float host_round_bf16(float x) {
  uint32_t u;
  memcpy(&u, &x, 4);
  if ((u & 0x7f800000u) == 0x7f800000u) return x;   // inf / nan unchanged
  u += 0x7fffu + ((u >> 16) & 1u);
  u &= 0xffff0000u;
  float r;
  memcpy(&r, &u, 4);
  return r;
}

}  // namespace qvl

using namespace qvl;

extern "C" {

const char* qvl_last_error(void) { return g_err; }

const char* qvl_status_string(int status) {
  switch (status) {
    case QVL_OK: return "ok";
    case QVL_ERR_INVALID_ARG: return "invalid argument";
    case QVL_ERR_UNSUPPORTED: return "unsupported";
    case QVL_ERR_MISALIGNED: return "misaligned";
    case QVL_ERR_WORKSPACE: return "workspace too small";
    case QVL_ERR_LAUNCH: return "launch failure";
  }
  return "unknown";
}

int qvl_version(void) { return 1; }

// ---------------------------------------------------------------------------------------------
// metadata
// ---------------------------------------------------------------------------------------------
int qvl_grid_counts(const int32_t* grid, int64_t n_grids, int32_t merge, int64_t* n_tokens, int64_t* n_segments) {
  if (!grid && n_grids > 0) return set_error(QVL_ERR_INVALID_ARG, "grid_thw is NULL");
  if (merge <= 0) return set_error(QVL_ERR_INVALID_ARG, "merge=%d", merge);
  int64_t nt = 0, ns = 0;
  for (int64_t i = 0; i < n_grids; ++i) {
    const int64_t t = grid[3 * i], h = grid[3 * i + 1], w = grid[3 * i + 2];
    if (t <= 0 || h <= 0 || w <= 0)
      return set_error(QVL_ERR_INVALID_ARG, "grid %lld: non-positive (t,h,w)=(%lld,%lld,%lld)", (long long)i,
                       (long long)t, (long long)h, (long long)w);
    if (h % merge || w % merge)
      return set_error(QVL_ERR_INVALID_ARG, "grid %lld: h=%lld, w=%lld not divisible by merge %d", (long long)i,
                       (long long)h, (long long)w, merge);
    nt += t * h * w;
    ns += t;
  }
  if (nt > (int64_t)INT32_MAX) return set_error(QVL_ERR_INVALID_ARG, "too many tokens: %lld", (long long)nt);
  if (n_tokens) *n_tokens = nt;
  if (n_segments) *n_segments = ns;
  return QVL_OK;
}

// model.py:686-693 (rotary ids), 713-739 + 761-764 (pos-embed taps), 831-834 (cu_seqlens).
int qvl_vision_metadata(const int32_t* grid, int64_t n_grids, int32_t merge, int32_t num_pos, int32_t dtype,
                        int32_t* cu, int32_t* pos_hw, int32_t* tap_idx, float* tap_w) {
  int64_t N = 0, S = 0;
  int rc = qvl_grid_counts(grid, n_grids, merge, &N, &S);
  if (rc) return rc;
  const int num_grid = (int)sqrt((double)num_pos);
  if (num_grid * num_grid != num_pos && (tap_idx || tap_w))
    return set_error(QVL_ERR_INVALID_ARG, "num_position_embeddings=%d is not a square", num_pos);
  if (cu) {
    int64_t s = 0, acc = 0;
    cu[s++] = 0;
    for (int64_t i = 0; i < n_grids; ++i)
      for (int32_t f = 0; f < grid[3 * i]; ++f) {
        acc += (int64_t)grid[3 * i + 1] * grid[3 * i + 2];
        cu[s++] = (int32_t)acc;
      }
  }
  int64_t off = 0;
  std::vector<double> hs, ws;
  std::vector<int32_t> hf, wf;
  std::vector<std::array<int64_t, 4>> done;   // (t, h, w, first token) of the grids computed so far
  for (int64_t i = 0; i < n_grids; ++i) {
    const int t = grid[3 * i], h = grid[3 * i + 1], w = grid[3 * i + 2];
    const int64_t n_tok = (int64_t)t * h * w;
    // A grid equal to an earlier one has the same per-token metadata: copy it (a batch of
    // same-size images builds one image's worth).
    int64_t src = -1;
    for (const auto& d : done)
      if (d[0] == t && d[1] == h && d[2] == w) { src = d[3]; break; }
    if (src >= 0) {
      if (pos_hw) memcpy(pos_hw + 2 * off, pos_hw + 2 * src, (size_t)n_tok * 2 * sizeof(int32_t));
      for (int j = 0; j < 4; ++j) {
        if (tap_idx) memcpy(tap_idx + j * N + off, tap_idx + j * N + src, (size_t)n_tok * sizeof(int32_t));
        if (tap_w) memcpy(tap_w + j * N + off, tap_w + j * N + src, (size_t)n_tok * sizeof(float));
      }
      off += n_tok;
      continue;
    }
    done.push_back({t, h, w, off});
    const int bw = w / merge;
    // np.linspace(0, num_grid-1, n, dtype=float32): float64 k*step, last = stop, cast to f32.
    auto linspace = [&](int n, std::vector<double>& val, std::vector<int32_t>& fl) {
      val.resize(n); fl.resize(n);
      const double stop = (double)(num_grid - 1);
      const double step = n > 1 ? stop / (double)(n - 1) : 0.0;
      for (int k = 0; k < n; ++k) {
        double y = (n > 1) ? (double)k * step : 0.0;
        if (n > 1 && k == n - 1) y = stop;
        const float y32 = (float)y;
        fl[k] = (int32_t)y32;                 // astype(int32): truncation
        val[k] = (double)y32 - (double)fl[k]; // f32 - int32 -> float64 (numpy promotion)
      }
    };
    if (tap_idx || tap_w) { linspace(h, hs, hf); linspace(w, ws, wf); }
    const int64_t hw = (int64_t)h * w;
    // Tokens in merge-block order, walked structurally (no per-token division): frame f, block row
    // hb, block column wb, then the merge x merge positions (mi, mj) of the block.
    int64_t tok = off;
    for (int f = 0; f < t; ++f)
      for (int hb = 0; hb < h / merge; ++hb)
        for (int wb = 0; wb < bw; ++wb)
          for (int mi = 0; mi < merge; ++mi)
            for (int mj = 0; mj < merge; ++mj, ++tok) {
              const int row = merge * hb + mi, col = merge * wb + mj;
              if (pos_hw) { pos_hw[2 * tok] = row; pos_hw[2 * tok + 1] = col; }
              if (!(tap_idx || tap_w)) continue;
              // jnp.repeat(.., t, axis=0) frame expansion: raster row (f*h*w + row*w + col) // t.
              int pr = row, pc = col;
              if (t > 1) {
                const int64_t src = (f * hw + (int64_t)row * w + col) / t;
                pr = (int)(src / w);
                pc = (int)(src - (int64_t)pr * w);
              }
              const int h0 = hf[pr], w0 = wf[pc];
              const int h1 = std::min(h0 + 1, num_grid - 1), w1 = std::min(w0 + 1, num_grid - 1);
              const double dh = hs[pr], dw = ws[pc];
              if (tap_idx) {
                tap_idx[0 * N + tok] = h0 * num_grid + w0;
                tap_idx[1 * N + tok] = h0 * num_grid + w1;
                tap_idx[2 * N + tok] = h1 * num_grid + w0;
                tap_idx[3 * N + tok] = h1 * num_grid + w1;
              }
              if (tap_w) {
                const double wv[4] = {(1.0 - dh) * (1.0 - dw), (1.0 - dh) * dw, dh * (1.0 - dw), dh * dw};
                for (int j = 0; j < 4; ++j) {
                  float v = (float)wv[j];
                  if (dtype == QVL_DTYPE_BF16) v = host_round_bf16(v);
                  tap_w[j * N + tok] = v;
                }
              }
            }
    off += (int64_t)t * hw;
  }
  return QVL_OK;
}

// model.py:769-799 (_get_window_index) and 828-830 (the full-attention cu_seqlens of the window
// branch, which scales token counts by merge_unit: its boundaries are clamped to n_tokens here as
// the reference's q[start:end] slicing clamps them).
int qvl_window_metadata(const int32_t* grid, int64_t n_grids, int32_t merge, int32_t patch_size, int32_t window_size,
                        int32_t* window_index, int32_t* cu_window, int64_t capacity, int64_t* n_cu_window,
                        int32_t* cu_full) {
  int64_t N = 0, S = 0;
  int rc = qvl_grid_counts(grid, n_grids, merge, &N, &S);
  if (rc) return rc;
  if (!n_cu_window) return set_error(QVL_ERR_INVALID_ARG, "window metadata: n_cu_window is NULL");
  if (patch_size <= 0) return set_error(QVL_ERR_INVALID_ARG, "patch_size=%d", patch_size);
  const int vw = window_size / merge / patch_size;   // vit_merger_window_size
  if (vw <= 0) return set_error(QVL_ERR_INVALID_ARG, "window_size=%d gives an empty window", window_size);
  const int64_t mm = (int64_t)merge * merge;
  std::vector<int32_t> cu(1, 0);
  int64_t wid = 0, k = 0;
  for (int64_t i = 0; i < n_grids; ++i) {
    const int64_t t = grid[3 * i], gh = grid[3 * i + 1] / merge, gw = grid[3 * i + 2] / merge;
    const int64_t nh = (gh + vw - 1) / vw, nw = (gw + vw - 1) / vw;
    for (int64_t f = 0; f < t; ++f)
      for (int64_t a = 0; a < nh; ++a)
        for (int64_t b = 0; b < nw; ++b) {
          int64_t len = 0;
          for (int64_t ih = 0; ih < vw; ++ih)
            for (int64_t iw = 0; iw < vw; ++iw) {
              const int64_t r = a * vw + ih, c = b * vw + iw;
              if (r >= gh || c >= gw) continue;              // the -100 padding
              if (window_index) window_index[k] = (int32_t)(wid + (f * gh + r) * gw + c);
              ++k;
              ++len;
            }
          const int32_t next = (int32_t)(cu.back() + len * mm);
          if (next != cu.back()) cu.push_back(next);          // consecutive duplicates dropped
        }
    wid += t * gh * gw;
  }
  *n_cu_window = (int64_t)cu.size();
  if (cu_window) {
    if (capacity < (int64_t)cu.size())
      return set_error(QVL_ERR_INVALID_ARG, "window metadata: cu_window capacity %lld < %lld", (long long)capacity,
                       (long long)cu.size());
    memcpy(cu_window, cu.data(), cu.size() * sizeof(int32_t));
  }
  if (cu_full) {
    int64_t acc = 0;
    cu_full[0] = 0;
    for (int64_t i = 0; i < n_grids; ++i) {
      acc += (int64_t)grid[3 * i] * grid[3 * i + 1] * grid[3 * i + 2] * mm;
      cu_full[i + 1] = (int32_t)std::min<int64_t>(acc, N);
    }
  }
  return QVL_OK;
}

// The plain work list of qvl_attention_worklist, built into `out` (4 ints per item).
static int build_worklist(const int32_t* cu, int64_t n_seg, int32_t num_heads, std::vector<int32_t>& out) {
  if (!cu) return set_error(QVL_ERR_INVALID_ARG, "cu_seqlens is NULL");
  if (num_heads <= 0) return set_error(QVL_ERR_INVALID_ARG, "num_heads=%d", num_heads);
  std::vector<std::pair<int32_t, int32_t>> segs;
  for (int64_t i = 0; i < n_seg; ++i) {
    if (cu[i + 1] < cu[i]) return set_error(QVL_ERR_INVALID_ARG, "cu_seqlens not monotone at %lld", (long long)i);
    if (cu[i + 1] > cu[i]) segs.push_back({cu[i], cu[i + 1]});
  }
  std::stable_sort(segs.begin(), segs.end(),
                   [](const std::pair<int32_t, int32_t>& a, const std::pair<int32_t, int32_t>& b) {
                     return (a.second - a.first) > (b.second - b.first);
                   });
  // (segment, head) groups, longest first, each to the queue with the least work so far
  // (work = query tiles x keys); a group's tiles stay in one queue so its K/V stay in one L2.
  std::vector<std::vector<std::array<int32_t, 4>>> queue(kAttnQueues);
  std::vector<int64_t> load(kAttnQueues, 0);
  for (auto& sg : segs) {
    const int32_t len = sg.second - sg.first;
    const int64_t ntile = (len + kAttnTileM - 1) / kAttnTileM;
    for (int32_t h = 0; h < num_heads; ++h) {
      int qi = 0;
      for (int j = 1; j < kAttnQueues; ++j)
        if (load[j] < load[qi]) qi = j;
      load[qi] += ntile * len;
      for (int32_t q0 = sg.first; q0 < sg.second; q0 += kAttnTileM) queue[qi].push_back({sg.first, sg.second, q0, h});
    }
  }
  size_t longest = 0;
  for (auto& q : queue) longest = std::max(longest, q.size());
  const int64_t n = (int64_t)longest * kAttnQueues;
  // Item k goes to the workgroup k, which the dispatcher places on XCD k % 8: queue k % 8,
  // position k / 8. Short queues are padded with empty items (start == end).
  out.assign(4 * (size_t)n, 0);
  for (int64_t k = 0; k < n; ++k) {
    const auto& q = queue[k % kAttnQueues];
    const size_t pos = (size_t)(k / kAttnQueues);
    if (pos < q.size())
      for (int c = 0; c < 4; ++c) out[4 * k + c] = q[pos][c];
  }
  return QVL_OK;
}

int qvl_attention_worklist(const int32_t* cu, int64_t n_seg, int32_t num_heads, int32_t* items, int64_t capacity,
                           int64_t* n_items) {
  if (!cu || !n_items) return set_error(QVL_ERR_INVALID_ARG, "cu_seqlens / n_items is NULL");
  std::vector<int32_t> list;
  QVL_TRY_RC(build_worklist(cu, n_seg, num_heads, list));
  const int64_t n = (int64_t)list.size() / 4;
  *n_items = n;
  if (!items) return QVL_OK;
  if (capacity < n) return set_error(QVL_ERR_INVALID_ARG, "worklist capacity %lld < %lld", (long long)capacity, (long long)n);
  std::copy(list.begin(), list.end(), items);
  return QVL_OK;
}

int qvl_attention_worklist_split(const int32_t* cu, int64_t n_seg, int32_t num_heads, int32_t head_dim,
                                 int32_t n_cus, int32_t* items, int64_t capacity, int64_t* n_items,
                                 int64_t* n_whole) {
  if (!n_items || !n_whole) return set_error(QVL_ERR_INVALID_ARG, "worklist_split: n_items / n_whole is NULL");
  if (head_dim != 64 && head_dim != 72 && head_dim != 80)
    return set_error(QVL_ERR_UNSUPPORTED, "worklist_split: head_dim=%d (supported: 64, 72, 80)", head_dim);
  if (n_cus <= 0) return set_error(QVL_ERR_INVALID_ARG, "worklist_split: n_cus=%d", n_cus);
  if (num_heads > kAttnHeadMask) return set_error(QVL_ERR_UNSUPPORTED, "worklist_split: num_heads=%d", num_heads);
  if (!cu) return set_error(QVL_ERR_INVALID_ARG, "cu_seqlens is NULL");
  std::vector<int32_t> base;
  QVL_TRY_RC(build_worklist(cu, n_seg, num_heads, base));
  const int64_t n = (int64_t)base.size() / 4;
  // The last round of workgroup slots: the kernels run 4 (head_dim 64) or 3 (72, 80) workgroups per
  // CU. When that round's items leave at least half of the CUs idle, each is split along its key
  // tiles into up to 8 parts (at least 2 tiles each) so that the parts fill the slots. A round
  // with one workgroup on most CUs is not split: a CU's lone workgroup runs faster than one of
  // four, and the parts' partial outputs and the combine cost more than the idle slots (MI355X,
  // 2304 items on 1024 slots: split 195 us, whole 190 us; 896 items on 768 slots: split 5.5 %
  // faster over the whole tower).
  const int64_t slots = (int64_t)n_cus * (head_dim == 64 ? 4 : 3);
  std::vector<int64_t> real;
  for (int64_t k = 0; k < n; ++k)
    if (base[4 * k + 1] > base[4 * k]) real.push_back(k);
  const int64_t nr = (int64_t)real.size();
  const int64_t t = nr >= slots ? nr % slots : nr;
  const int64_t f = t > 0 && 2 * t <= n_cus ? std::min<int64_t>(kAttnMaxSplit, slots / t) : 1;
  std::vector<std::pair<int64_t, int>> tail;     // (item, parts)
  if (f >= 2) {
    for (int64_t i = nr - t; i < nr; ++i) {
      const int64_t k = real[i];
      const int32_t s0 = base[4 * k], s1 = base[4 * k + 1];
      const int64_t n_kt = (s1 - (s0 & ~63) + 63) / 64;
      const int parts = (int)std::min<int64_t>(f, n_kt / 2);
      if (parts >= 2) tail.push_back({k, parts});
    }
  }
  int64_t total = n;
  for (auto& tp : tail) total += tp.second;
  *n_whole = n;
  *n_items = total;
  if (!items) return QVL_OK;
  if (capacity < total)
    return set_error(QVL_ERR_INVALID_ARG, "worklist_split capacity %lld < %lld", (long long)capacity, (long long)total);
  std::copy(base.begin(), base.begin() + 4 * n, items);
  int64_t w = n;
  for (auto& tp : tail) {
    const int32_t* it = &base[4 * tp.first];
    for (int sp = 0; sp < tp.second; ++sp, ++w) {
      items[4 * w] = it[0];
      items[4 * w + 1] = it[1];
      items[4 * w + 2] = it[2];
      items[4 * w + 3] = it[3] | (sp << kAttnSplitShift) | (tp.second << kAttnPartsShift);
    }
    for (int c = 0; c < 4; ++c) items[4 * tp.first + c] = 0;   // the whole item leaves the main list
  }
  return QVL_OK;
}

int qvl_rotary_inv_freq(int32_t head_dim, float theta, float* inv) {
  if (head_dim <= 0 || head_dim % 4 || head_dim > 128 || !inv)
    return set_error(QVL_ERR_INVALID_ARG, "head_dim=%d", head_dim);
  const int dim = head_dim / 2;
  // 1.0 / (theta ** (arange(0, dim, 2, f32) / dim)) (model.py:544): the f32 exponent as the
  // reference forms it, the power in double, one rounding to f32 (XLA's f32 pow is not
  // reproducible bit for bit on the host; this is within 1 ulp of it and of numpy's).
  for (int j = 0; j < head_dim / 4; ++j) {
    const float e = (float)(2 * j) / (float)dim;
    inv[j] = (float)(1.0 / pow((double)theta, (double)e));
  }
  return QVL_OK;
}

}  // extern "C"
