// Host-side helpers shared by the C-ABI entry points: error reporting and argument checks.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "flashdmla.h"

namespace dmla {

// Records a printf-style message for dmla_last_error() and returns `code`.
int fail(int code, const char* fmt, ...) __attribute__((format(printf, 2, 3)));

// Clears the thread's error message; every entry point calls it first.
void clear_error();

// Converts a pending launch error into DMLA_ERR_HIP.
int check_launch(const char* what);

inline bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }
inline bool mult8(int64_t s) { return (s % 8) == 0; }

// Number of compute units of the current device (cached per device).
int device_cu_count();

// Split-KV combine (dmla_cache.hip): part_o [.., split, .., d] fp32 partial outputs, each
// normalised over its split, and part_lse natural-log sums, addressed by element strides.
// The split count of sequence b is num_splits[b] (at most max_splits) when given, else
// derived from seqlens[b] and pages_per_split when given, else max_splits.  Split s of
// sequence b is at b * sb + s * ss, or at (split_base[b] + s) * ss when split_base is given.
// skip_single leaves sequences with one split untouched (their rows were written by the
// producer directly).
// part_o16, when set, replaces part_o with bf16 partials of the same layout (the decode's own).
struct CombineArgs {
  const float* part_o;
  const __bf16* part_o16;
  const float* part_lse;
  const int32_t* num_splits;
  const int32_t* split_base;
  const int32_t* seqlens;
  __bf16* o;
  float* lse;                 // nullable, [B, H] contiguous
  int B, H, max_splits, d;
  int pages_per_split, page_size, max_pages;
  int skip_single;
  int64_t po_sb, po_ss, po_sh, lse_sb, lse_ss, lse_sh, o_sb, o_sh;
};
int launch_lse_combine(const CombineArgs& a, hipStream_t stream, const char* what);

}  // namespace dmla
