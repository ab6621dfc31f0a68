// nuq_launch.h -- launch helpers shared by the compact pack and unpack
// sources (host side) and the wave-level LDS ordering both use.
#pragma once

#include "nuq_core.h"

namespace {

constexpr int kThreads = 256;
constexpr int kBatchItems = 16;  // tensors per batched pack / unpack launch

HKV_DEV void wave_sync() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

bool pow2_G(int D) { return D % 8 == 0 && D >= 8 && D <= 256 && ((D / 8) & (D / 8 - 1)) == 0; }

int num_cus() {
  static int n = 0;
  if (!n) {
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess ||
        hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0)
      n = 256;
  }
  return n;
}

// Persistent grid: as many blocks as fit on the device at once (at most one
// per tile).
template <typename K>
unsigned resident_grid(K kernel, int64_t nblocks, size_t lds = 0) {
  int per_cu = 0;
  if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, kernel, kThreads, lds) != hipSuccess ||
      per_cu < 1)
    per_cu = 1;
  return (unsigned)std::min<int64_t>(nblocks, (int64_t)per_cu * num_cus());
}


}  // namespace
