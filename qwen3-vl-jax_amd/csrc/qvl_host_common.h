// Host-side constants and error plumbing shared by every libqvl source (plain C++, no HIP headers,
// so qvl_meta.cpp also builds as ordinary C++ for the CPU sanitizer run).
#pragma once
#include <stdint.h>

#include "qvl_vision.h"

namespace qvl {

// Records a message for qvl_last_error() on the calling thread and returns `code`.
int set_error(int code, const char* fmt, ...);

#define QVL_TRY_RC(expr) do { int _rc = (expr); if (_rc) return _rc; } while (0)

constexpr int kAttnTileM = 128;   // query tile height of the attention kernels
constexpr int kAttnQueues = 8;    // attention work queues: one per XCD of an MI355X

// Attention work item head field (the 4th int of a work item): the head in bits 0..11; for a
// part of a split item, the part index in bits 12..19 and the part count in bits 20..27 (both 0
// for whole items). A part covers key tiles [n_kt*i/parts, n_kt*(i+1)/parts) of its segment and
// writes its unnormalised output and softmax state to partial slot (item - n_whole); the combine
// kernel then writes the item's output.
constexpr int kAttnHeadMask = 0xfff, kAttnSplitShift = 12, kAttnPartsShift = 20, kAttnMaxSplit = 8;

}  // namespace qvl
