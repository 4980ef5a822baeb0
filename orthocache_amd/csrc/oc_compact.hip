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
#include "oc_kernels.h"

namespace oc {

__device__ __forceinline__ bool keep_one(const CompactParams& p, int gj, int h, float tau, float zmax) {
  if (p.mask_in) {
    const int mh = p.mask_in_heads;
    return p.mask_in[(int64_t)gj * mh + (mh == 1 ? 0 : h)] != 0;
  }
  const int64_t e = (int64_t)gj * p.num_kv_heads + h;
  float tm = p.tau_max[e];
  for (int i = 1; i < p.tau_parts; ++i)
    tm = nanmax(tm, p.tau_max[(int64_t)i * p.total_blocks * p.num_kv_heads + e]);
  bool k = tm >= tau;  // false for NaN on either side
  if (p.zeta) k = k && (p.zeta[e] <= zmax);
  return k;
}

__device__ __forceinline__ bool keep_any(const CompactParams& p, int gj, float tau, float zmax) {
  const int nh = (p.mask_in && p.mask_in_heads == 1) ? 1 : p.num_kv_heads;
  bool a = false;
  for (int h = 0; h < nh; ++h) a = a || keep_one(p, gj, h, tau, zmax);
  return a;
}

// Exclusive prefix of `pred` over the workgroup and the total.  Uniform call.
__device__ __forceinline__ int block_scan_bool(bool pred, int* s_cnt, int& total) {
  const int lane = threadIdx.x & (kWave - 1);
  const int wave = threadIdx.x / kWave;
  const int nwaves = blockDim.x / kWave;
  const unsigned long long bal = __ballot(pred);
  const int in_wave = __popcll(bal & ((1ull << lane) - 1ull));
  if (lane == 0) s_cnt[wave] = __popcll(bal);
  __syncthreads();
  int before = 0, tot = 0;
  for (int w = 0; w < nwaves; ++w) {
    const int c = s_cnt[w];
    before += (w < wave) ? c : 0;
    tot += c;
  }
  __syncthreads();
  total = tot;
  return before + in_wave;
}

template <typename Pred>
__device__ __forceinline__ int stable_partition(int nb, int* out, Pred pred, int* s_cnt) {
  const int t = threadIdx.x;
  int n = 0;
  for (int base = 0; base < nb; base += blockDim.x) {
    const int j = base + t;
    const bool a = (j < nb) && pred(j);
    int tot;
    block_scan_bool(a, s_cnt, tot);
    n += tot;
  }
  int run_act = 0, run_in = 0;
  for (int base = 0; base < nb; base += blockDim.x) {
    const int j = base + t;
    const bool a = (j < nb) && pred(j);
    int tot;
    const int ex = block_scan_bool(a, s_cnt, tot);
    if (j < nb) {
      const int pos = a ? (run_act + ex) : (n + run_in + (t - ex));
      out[pos] = j;
    }
    const int valid = min((int)blockDim.x, nb - base);
    run_act += tot;
    run_in += valid - tot;
  }
  return n;
}

__global__ __launch_bounds__(256) void compact_kernel(CompactParams p) {
  __shared__ int s_cnt[16];
  const int seg = blockIdx.x;
  const int off = p.cu_blocks ? p.cu_blocks[seg] : 0;
  const int nb = p.cu_blocks ? p.cu_blocks[seg + 1] - off : p.nb_single;
  const float tau = p.tau_arr ? p.tau_arr[seg] : p.tau;
  const float zmax = p.zmax_arr ? p.zmax_arr[seg] : p.zeta_max;
  const int H = p.num_kv_heads;
  const int t = threadIdx.x;

  if (p.mask_out || p.active_out) {
    for (int j = t; j < nb; j += blockDim.x) {
      bool any = false;
      for (int h = 0; h < H; ++h) {
        const bool k = keep_one(p, off + j, h, tau, zmax);
        if (p.mask_out) p.mask_out[(int64_t)(off + j) * H + h] = k ? 1 : 0;
        any = any || k;
      }
      if (p.active_out) p.active_out[off + j] = any ? 1 : 0;
    }
  }

  if (p.indices) {
    const int n = stable_partition(
        nb, p.indices + off, [&](int j) { return keep_any(p, off + j, tau, zmax); }, s_cnt);
    if (t == 0 && p.num_active) p.num_active[seg] = n;
  }

  if (p.head_indices) {
    for (int h = 0; h < H; ++h) {
      int* out = p.head_indices + (int64_t)h * p.total_blocks + off;
      int n = stable_partition(
          nb, out, [&](int j) { return keep_one(p, off + j, h, tau, zmax); }, s_cnt);
      bool uniform = false;
      if (n == 0 && p.empty_head_all) {
        for (int j = t; j < nb; j += blockDim.x) out[j] = j;
        n = nb;
        uniform = true;
      }
      if (t == 0) {
        p.head_num_active[seg * H + h] = n;
        if (p.head_uniform) p.head_uniform[seg * H + h] = uniform ? 1 : 0;
      }
    }
  }
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
