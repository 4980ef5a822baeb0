// Two-gate mask and stream compaction.
//
// Replaces the mask step of compute_multiband_mask
// (src/orthocache/spectral_energy.py:180-234) and the index part of
// stream_compact (src/orthocache/compaction.py:65-82,
// src/orthocache/adaptive_attention.py:29-40):
//   keep[j,h]  = (tau_max[j,h] >= tau) && (zeta[j,h] <= zeta_max)   (NaN -> false)
//   active[j]  = OR_h keep[j,h]
//   indices    = stable partition of 0..nb-1: active blocks ascending, then
//                inactive blocks ascending (the full permutation)
//   num_active = popcount(active)
// All on device, no host synchronisation.  One workgroup per segment (a
// sequence of a ragged batch or a layer of a multi-layer sweep); the
// partition is a wave ballot + mbcnt prefix, combined across waves in LDS.
// Optionally the same partition per kv head, for per-head attention.
#include "oc_compact_dev.h"

namespace oc {

constexpr int kFlagBytes = 16384;  // per-(block, head) keep flags of one chunk of blocks
constexpr int kActCap = 16384;     // per-block active flags kept in LDS for segments up to this size

__global__ __launch_bounds__(256) void compact_kernel(CompactParams p) {
  __shared__ uint8_t s_flag[kFlagBytes];
  __shared__ uint8_t s_act[kActCap];
  __shared__ int s_cnt[16];
  compact_segment(p, blockIdx.x, s_flag, kFlagBytes, s_act, kActCap, s_cnt);
}

// Block copy for the materialised compaction API (compaction.py:86-98,
// :103-154).  gather: dst[i] = src[idx[i]] for i < n, zero for i >= n.
// scatter: dst[idx[i]] = src[i] for i < n, zero for i >= n.  Blocks are
// contiguous runs of block_bytes (layout (seq, heads, dim)).
__global__ __launch_bounds__(256) void copy_blocks_kernel(CopyParams p) {
  const int i = blockIdx.y;
  const int n = *p.num_active;
  const int idx = p.indices[i];
  const bool live = i < n;
  const int64_t src_blk = p.scatter ? i : idx;
  const int64_t dst_blk = p.scatter ? idx : i;
  const uint4* s = reinterpret_cast<const uint4*>(reinterpret_cast<const char*>(p.src) + src_blk * p.block_bytes);
  uint4* d = reinterpret_cast<uint4*>(reinterpret_cast<char*>(p.dst) + dst_blk * p.block_bytes);
  const int64_t nvec = p.block_bytes / 16;
  for (int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; e < nvec; e += (int64_t)gridDim.x * blockDim.x) {
    d[e] = live ? s[e] : make_uint4(0u, 0u, 0u, 0u);
  }
}

hipError_t launch_compact(const CompactParams& p, hipStream_t s) {
  if (p.num_segments == 0) return hipSuccess;
  hipLaunchKernelGGL(compact_kernel, dim3(p.num_segments), dim3(256), 0, s, p);
  return hipGetLastError();
}

hipError_t launch_copy_blocks(const CopyParams& p, hipStream_t s) {
  if (p.num_blocks == 0) return hipSuccess;
  const int64_t nvec = p.block_bytes / 16;
  int gx = (int)((nvec + 255) / 256);
  if (gx > 64) gx = 64;
  hipLaunchKernelGGL(copy_blocks_kernel, dim3(gx, p.num_blocks), dim3(256), 0, s, p);
  return hipGetLastError();
}

}  // namespace oc
