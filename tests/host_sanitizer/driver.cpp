// CPU sanitizer driver for libqvl's GPU-free host code (qvl_meta.cpp): exercises the metadata,
// window and work-list entries on random and malformed inputs with exactly-sized buffers, so that
// AddressSanitizer / UBSan see every out-of-bounds write or undefined operation. Exit 0 = clean.
#include <stdio.h>
#include <stdlib.h>

#include <random>
#include <vector>

#include "qvl_vision.h"

static int failures = 0;
#define CHECK(cond, ...)                                  \
  do {                                                    \
    if (!(cond)) {                                        \
      fprintf(stderr, "CHECK failed %s:%d: ", __FILE__, __LINE__); \
      fprintf(stderr, __VA_ARGS__);                       \
      fprintf(stderr, "\n");                              \
      ++failures;                                         \
    }                                                     \
  } while (0)

static void one_grid_set(std::mt19937& rng, const std::vector<int32_t>& g, int merge) {
  const int64_t ng = (int64_t)g.size() / 3;
  int64_t N = -1, S = -1;
  int rc = qvl_grid_counts(g.data(), ng, merge, &N, &S);
  if (rc) return;   // rejected grid: nothing more to check
  const int npos = 2304;
  std::vector<int32_t> cu(S + 1), pos(2 * N), idx(4 * N);
  std::vector<float> w(4 * N);
  rc = qvl_vision_metadata(g.data(), ng, merge, npos, QVL_DTYPE_BF16, cu.data(), pos.data(), idx.data(), w.data());
  CHECK(rc == QVL_OK, "metadata rc=%d", rc);
  for (int64_t s = 0; s < S; ++s) CHECK(cu[s + 1] > cu[s], "cu not increasing");
  CHECK(cu[S] == N, "cu end");
  for (int64_t i = 0; i < 4 * N; ++i) CHECK(idx[i] >= 0 && idx[i] < npos, "tap index %d", idx[i]);
  // metadata without the pos-embed table
  rc = qvl_vision_metadata(g.data(), ng, merge, 0, QVL_DTYPE_F32, cu.data(), pos.data(), nullptr, nullptr);
  CHECK(rc == QVL_OK, "metadata without taps rc=%d", rc);
  // work lists, exact capacity and one short
  for (int heads : {1, 3, 16}) {
    int64_t n = 0;
    CHECK(qvl_attention_worklist(cu.data(), S, heads, nullptr, 0, &n) == QVL_OK, "worklist count");
    std::vector<int32_t> items(4 * n);
    CHECK(qvl_attention_worklist(cu.data(), S, heads, items.data(), n, &n) == QVL_OK, "worklist fill");
    if (n > 0) {
      std::vector<int32_t> small(4 * (n - 1));
      CHECK(qvl_attention_worklist(cu.data(), S, heads, small.data(), n - 1, &n) != QVL_OK, "short capacity");
    }
    // every (query tile, head) once
    std::vector<int> seen((size_t)N * heads, 0);
    for (int64_t k = 0; k < n; ++k) {
      const int32_t s0 = items[4 * k], s1 = items[4 * k + 1], q0 = items[4 * k + 2], h = items[4 * k + 3];
      if (s1 <= s0) continue;
      for (int32_t q = q0; q < q0 + 128 && q < s1; ++q) seen[(size_t)q * heads + h]++;
    }
    for (size_t i = 0; i < seen.size(); ++i) CHECK(seen[i] == 1, "query/head %zu covered %d times", i, seen[i]);
    for (int hd : {64, 72}) {
      const int n_cus = 1 + (int)(rng() % 300);
      int64_t ns = 0, nw = 0;
      CHECK(qvl_attention_worklist_split(cu.data(), S, heads, hd, n_cus, nullptr, 0, &ns, &nw) == QVL_OK, "split count");
      std::vector<int32_t> sp(4 * ns);
      CHECK(qvl_attention_worklist_split(cu.data(), S, heads, hd, n_cus, sp.data(), ns, &ns, &nw) == QVL_OK,
            "split fill");
      CHECK(nw <= ns, "n_whole");
    }
  }
  // window metadata: count, exact fill, short capacity
  for (int window : {32, 64, 112}) {
    int64_t ncw = 0;
    if (qvl_window_metadata(g.data(), ng, merge, 16, window, nullptr, nullptr, 0, &ncw, nullptr)) continue;
    std::vector<int32_t> widx(N / (merge * merge)), cuw(ncw), cuf(ng + 1);
    CHECK(qvl_window_metadata(g.data(), ng, merge, 16, window, widx.data(), cuw.data(), ncw, &ncw, cuf.data()) ==
              QVL_OK, "window fill");
    if (ncw > 1) {
      std::vector<int32_t> small(ncw - 1);
      CHECK(qvl_window_metadata(g.data(), ng, merge, 16, window, nullptr, small.data(), ncw - 1, &ncw, nullptr) !=
                QVL_OK, "window short capacity");
    }
  }
}

int main() {
  std::mt19937 rng(1234);
  int cases = 0;
  for (int it = 0; it < 300; ++it) {
    const int ng = 1 + (int)(rng() % 4);
    std::vector<int32_t> g;
    for (int i = 0; i < ng; ++i) {
      int t = 1 + (int)(rng() % 3), h = 2 * (1 + (int)(rng() % 20)), w = 2 * (1 + (int)(rng() % 20));
      if (it % 37 == 5) h += 1;          // malformed: odd side
      if (it % 53 == 7) t = 0;           // malformed: empty frame count
      g.insert(g.end(), {t, h, w});
    }
    one_grid_set(rng, g, 2);
    ++cases;
  }
  // malformed arguments: each must return an error, not write anywhere
  int64_t n = 0, s = 0;
  const int32_t grid[3] = {1, 4, 4};
  CHECK(qvl_grid_counts(nullptr, 1, 2, &n, &s) != QVL_OK, "NULL grid");
  CHECK(qvl_grid_counts(grid, 1, 0, &n, &s) != QVL_OK, "merge 0");
  CHECK(qvl_vision_metadata(grid, 1, 2, 2300, QVL_DTYPE_BF16, nullptr, nullptr, (int32_t*)&n, nullptr) != QVL_OK,
        "non-square table");
  CHECK(qvl_attention_worklist(nullptr, 1, 4, nullptr, 0, &n) != QVL_OK, "NULL cu");
  CHECK(qvl_attention_worklist(grid, 1, 0, nullptr, 0, &n) != QVL_OK, "0 heads");
  const int32_t bad_cu[3] = {0, 8, 4};
  CHECK(qvl_attention_worklist(bad_cu, 2, 4, nullptr, 0, &n) != QVL_OK, "non-monotone cu");
  int64_t nw = 0;
  CHECK(qvl_attention_worklist_split(grid, 1, 4, 96, 8, nullptr, 0, &n, &nw) != QVL_OK, "head_dim 96");
  CHECK(qvl_attention_worklist_split(grid, 1, 4, 80, 8, nullptr, 0, &n, &nw) == QVL_OK, "head_dim 80");
  CHECK(qvl_window_metadata(grid, 1, 2, 16, 8, nullptr, nullptr, 0, &n, nullptr) != QVL_OK, "window < patch*merge");
  float inv[32];
  CHECK(qvl_rotary_inv_freq(128, 10000.f, inv) == QVL_OK, "inv_freq 128");
  CHECK(qvl_rotary_inv_freq(130, 10000.f, inv) != QVL_OK, "inv_freq 130");
  CHECK(qvl_last_error()[0] != 0, "error message");
  printf("host sanitizer driver: %d grid sets, %d failures\n", cases, failures);
  return failures ? 1 : 0;
}
