// Host-only parts of the C ABI declared in include/sparton.h.
#include "../../include/sparton.h"

#define SPARTON_EXPORT extern "C" __attribute__((visibility("default")))

namespace {
constexpr int kAbiVersion = 10;
// The backward takes any S and B with B * S and B * V below 2^31 (it runs its dH passes
// over windows of positions and chunks of batch rows).
constexpr int64_t kMaxBwdSeq = INT32_MAX;
constexpr int64_t kMaxBwdBatch = INT32_MAX;
}  // namespace

SPARTON_EXPORT const char* sparton_strerror(int code) {
  switch (code) {
    case SPARTON_OK: return "success";
    case SPARTON_EINVAL: return "invalid argument (null pointer, negative size, bad dtype, or D not a multiple of 16 bytes)";
    case SPARTON_EALIGN: return "a tensor base pointer is not 16-byte aligned (workspace: 256-byte)";
    case SPARTON_EUNSUPPORTED: return "shape outside the supported range (see sparton_limits)";
    case SPARTON_EWORKSPACE: return "workspace missing or smaller than sparton_fwd/bwd_workspace_bytes()";
    case SPARTON_ESCRATCH: return "sizes need more workspace than sparton_fwd_noalloc's static scratch (sparton_fwd_noalloc_max_workspace() bytes); use sparton_fwd with a workspace";
    default: return code > 0 ? "HIP kernel launch failed (code is the hipError_t)" : "unknown sparton status";
  }
}

SPARTON_EXPORT void sparton_limits(int64_t* max_bwd_seq, int64_t* max_bwd_batch) {
  if (max_bwd_seq) *max_bwd_seq = kMaxBwdSeq;
  if (max_bwd_batch) *max_bwd_batch = kMaxBwdBatch;
}

SPARTON_EXPORT int sparton_abi_version(void) { return kAbiVersion; }
