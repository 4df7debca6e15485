// rte_pack_index_noalloc: the deterministic pack of rte_pack_index with its histogram
// workspace in a file-scope device array instead of a caller- or library-allocated buffer,
// for callers that cannot allocate device memory (HIP graph capture, serving loops).
//
// The array is resolved to a device address once per device with hipGetSymbolAddress (the
// host-side name of a __device__ array is not a device address) and that address is what the
// kernels receive.  Every call on a device shares that device's array: calls that overlap on
// one device (different streams, or different host threads) race.  The pack's count kernel
// overwrites every histogram entry it later reads, so the array needs no clearing between
// calls.
#include "../../include/rte_hip.h"
#include "common.hpp"

#include <mutex>

namespace rte {
size_t pack_workspace_bytes(int P, int C);
int pack_pairs(const int32_t* cl, int P, int C, int k, const float* w, int32_t* offsets,
               int32_t* tok_of_slot, int32_t* pair_of_slot, int32_t* slot_of_pair, float* w_of_slot,
               int32_t* invalid, void* ws, size_t ws_bytes, hipStream_t s);
}  // namespace rte

namespace {

constexpr size_t kScratchBytes = size_t(1) << 20;  // 1 MiB per device
constexpr int kMaxDevices = 64;

__device__ __align__(256) int32_t scratch[kScratchBytes / sizeof(int32_t)];

std::mutex g_mu;
void* g_scratch[kMaxDevices] = {};

// Device address of this device's copy of `scratch` (resolved on the first call per device).
int scratch_ptr(void** out) {
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) {
    rte::set_error("pack_index_noalloc: hipGetDevice failed: %s", hipGetErrorString(e));
    return (int)e;
  }
  if (dev < 0 || dev >= kMaxDevices) {
    rte::set_error("pack_index_noalloc: device index %d outside [0, %d)", dev, kMaxDevices);
    return -1;
  }
  std::lock_guard<std::mutex> lock(g_mu);
  if (g_scratch[dev] == nullptr) {
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || p == nullptr) {
      rte::set_error("pack_index_noalloc: hipGetSymbolAddress(scratch) failed on device %d: %s", dev,
                     hipGetErrorString(e));
      return e != hipSuccess ? (int)e : -1;
    }
    g_scratch[dev] = p;
  }
  *out = g_scratch[dev];
  return 0;
}

}  // namespace

extern "C" {

size_t rte_pack_index_noalloc_max_bytes(void) { return kScratchBytes; }

int rte_pack_index_noalloc(const int32_t* cl, int P, int C, int k, const float* w, int32_t* offsets,
                           int32_t* tok_of_slot, int32_t* pair_of_slot, int32_t* slot_of_pair, float* w_of_slot,
                           int32_t* invalid, void* stream) {
  if (P < 0 || C < 1 || k < 1) {
    rte::set_error("pack_index_noalloc: bad sizes (P=%d, C=%d, k=%d)", P, C, k);
    return -1;
  }
  const size_t need = rte::pack_workspace_bytes(P, C);
  if (need > kScratchBytes) {
    rte::set_error("pack_index_noalloc: P=%d pairs over C=%d clusters need %zu bytes of scratch, more than the "
                   "%zu-byte static array; use rte_pack_index with a workspace",
                   P, C, need, kScratchBytes);
    return -1;
  }
  void* ws = nullptr;
  const int rc = scratch_ptr(&ws);
  if (rc != 0) return rc;
  return rte::pack_pairs(cl, P, C, k, w, offsets, tok_of_slot, pair_of_slot, slot_of_pair, w_of_slot, invalid, ws,
                         kScratchBytes, static_cast<hipStream_t>(stream));
}

}  // extern "C"
