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

// A list entry as NumPy-style indexing reads it: -nb <= i < 0 counts from
// the end.  Entries still outside [0, nb) are returned as is.
__device__ __forceinline__ int wrap_index(int i, int nb) { return (i < 0 && i >= -nb) ? i + nb : i; }

// Block copy for the materialised compaction API (compaction.py:86-98,
// :103-154).  Blocks are contiguous runs of block_bytes (layout (seq, heads,
// dim)); workgroup row blockIdx.y owns destination block j, so every
// destination block is written exactly once, whatever the list holds.
//  gather:  dst[j] = src[idx[j]] for j < n, zero for j >= n.  An entry
//           outside [0, nb) is clamped into it (JAX clamps gather indices).
//  scatter: dst[j] = src[i] for the largest i < n with idx[i] == j, zero when
//           no such i exists.  Entries outside [0, nb) are dropped (JAX drops
//           out-of-bounds scatter updates).  For a permutation this is
//           dst[idx[i]] = src[i] for i < n; for duplicate entries, whose
//           order a JAX scatter leaves to the implementation, the last list
//           position wins.
__global__ __launch_bounds__(256) void copy_blocks_kernel(CopyParams p) {
  __shared__ int s_owner[4];
  const int j = blockIdx.y;
  const int nb = p.num_blocks;
  int n = *p.num_active;
  n = n < 0 ? 0 : (n > nb ? nb : n);
  int src_blk = -1;
  if (!p.scatter) {
    if (j < n) {
      const int s = wrap_index(p.indices[j], nb);
      src_blk = s < 0 ? 0 : (s >= nb ? nb - 1 : s);
    }
  } else {
    // Each thread keeps its last matching position; positions rise with the
    // loop, so the maxima over threads and waves give the last one overall.
    int own = -1;
    for (int i = threadIdx.x; i < n; i += blockDim.x)
      if (wrap_index(p.indices[i], nb) == j) own = i;
    for (int off = 32; off > 0; off >>= 1) own = max(own, __shfl_xor(own, off, 64));
    if ((threadIdx.x & 63) == 0) s_owner[threadIdx.x >> 6] = own;
    __syncthreads();
    src_blk = max(max(s_owner[0], s_owner[1]), max(s_owner[2], s_owner[3]));
  }
  const bool live = src_blk >= 0;
  const uint4* s = reinterpret_cast<const uint4*>(reinterpret_cast<const char*>(p.src) +
                                                  (int64_t)(live ? src_blk : 0) * p.block_bytes);
  uint4* d = reinterpret_cast<uint4*>(reinterpret_cast<char*>(p.dst) + (int64_t)j * p.block_bytes);
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
