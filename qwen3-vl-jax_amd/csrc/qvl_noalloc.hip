// Allocation-free variant of the split attention entry: its partial-output scratch lives in a
// file-scope device array instead of a caller workspace, for callers that cannot allocate device
// memory (code under HIP graph capture, tight serving loops, harnesses that forbid hipMalloc).
#include <atomic>
#include <mutex>

#include "qvl_kernels.h"

namespace qvl {

// The split parts' partial outputs (unnormalised O, running max and row sum per query row):
// up to one part per workgroup slot, 4 slots per CU on a 256-CU MI355X at head_dim 72 needs
// 1024 * 128 * 74 * 4 B = 38.8 MB. Each GPU that runs this entry holds its own copy of the array
// until the process ends.
constexpr size_t kNoAllocScratchBytes = 40u << 20;
static __device__ __align__(256) unsigned char scratch[kNoAllocScratchBytes];

constexpr int kMaxDevices = 64;

// Device address of `scratch` on the current device. The host-side name `scratch` is only a
// stand-in for the symbol: kernels and copies take this address. Looked up once per device
// (with that device current) and kept.
static int scratch_ptr(void** out) {
  static std::once_flag once[kMaxDevices];
  static std::atomic<void*> ptr[kMaxDevices];
  static std::atomic<int> rc[kMaxDevices];
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices)
    return set_error(QVL_ERR_LAUNCH, "no-alloc scratch: no current device (or device id %d >= %d)", dev, kMaxDevices);
  std::call_once(once[dev], [dev] {
    void* p = nullptr;
    const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    rc[dev].store((int)e, std::memory_order_relaxed);
    ptr[dev].store(e == hipSuccess ? p : nullptr, std::memory_order_release);
  });
  void* p = ptr[dev].load(std::memory_order_acquire);
  if (!p)
    return set_error(QVL_ERR_LAUNCH, "no-alloc scratch: hipGetSymbolAddress failed on device %d: %s", dev,
                     hipGetErrorString((hipError_t)rc[dev].load(std::memory_order_relaxed)));
  *out = p;
  return QVL_OK;
}

}  // namespace qvl

using namespace qvl;

extern "C" {

size_t qvl_noalloc_scratch_bytes(void) { return kNoAllocScratchBytes; }

int qvl_attention_headmajor_split_noalloc(void* stream, int32_t dtype, const void* q, const void* k, const void* vt,
                                          const int32_t* tiles, int64_t n_tiles, int64_t n_whole, int64_t n_tokens,
                                          int32_t H, int32_t hd, void* out, int64_t ld_out) {
  size_t need = 0;
  if (n_tiles >= 0 && n_whole >= 0 && n_whole <= n_tiles && (hd == 64 || hd == 72 || hd == 80)) {
    int rc = qvl_attention_split_workspace_size(hd, n_tiles, n_whole, &need);
    if (rc) return rc;
    if (need > kNoAllocScratchBytes)
      return set_error(QVL_ERR_WORKSPACE,
                       "attention split (no-alloc): %lld parts need %zu bytes of scratch, above the %zu-byte maximum",
                       (long long)(n_tiles - n_whole), need, kNoAllocScratchBytes);
  }
  void* p = nullptr;
  if (need) {
    int rc = scratch_ptr(&p);
    if (rc) return rc;
  }
  // every argument check of the workspace entry applies; the scratch is its workspace
  return qvl_attention_headmajor_split(stream, dtype, q, k, vt, tiles, n_tiles, n_whole, n_tokens, H, hd, out, ld_out,
                                       p, p ? kNoAllocScratchBytes : 0);
}

}  // extern "C"
