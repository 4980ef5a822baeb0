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
  if (p.zeta) k = k & (p.zeta[e] <= zmax);
  return k;
}

// OR over heads without short-circuit, so the loads of all heads are in flight together.
__device__ __forceinline__ bool keep_any(const CompactParams& p, int gj, float tau, float zmax) {
  const int nh = (p.mask_in && p.mask_in_heads == 1) ? 1 : p.num_kv_heads;
  bool a = false;
#pragma unroll 8
  for (int h = 0; h < nh; ++h) a |= keep_one(p, gj, h, tau, zmax);
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

constexpr int kFlagBytes = 16384;  // per-(block, head) keep flags of one chunk of blocks
constexpr int kActCap = 16384;     // per-block active flags kept in LDS for segments up to this size

__global__ __launch_bounds__(256) void compact_kernel(CompactParams p) {
  __shared__ uint8_t s_flag[kFlagBytes];
  __shared__ uint8_t s_act[kActCap];
  __shared__ int s_cnt[16];
  const int seg = blockIdx.x;
  const int off = p.cu_blocks ? p.cu_blocks[seg] : 0;
  const int nb = p.cu_blocks ? p.cu_blocks[seg + 1] - off : p.nb_single;
  const float tau = p.tau_arr ? p.tau_arr[seg] : p.tau;
  const float zmax = p.zmax_arr ? p.zmax_arr[seg] : p.zeta_max;
  const int H = p.num_kv_heads;
  const int t = threadIdx.x;
  const bool act_in_lds = nb <= kActCap;
  const int cb = min((int)blockDim.x, kFlagBytes / H);  // blocks per chunk

  // Pass 1: every (block, head) predicate in parallel (coalesced), masks,
  // per-block OR through LDS, and the active count.  Each thread first loads
  // kEpt entries into registers (indices clamped, no branches) so the loads
  // are in flight together, then evaluates them.
  constexpr int kEpt = 8;
  int n = 0;
  if (p.indices || p.mask_out || p.active_out) {
    const float* zsrc = p.zeta ? p.zeta : p.tau_max;  // dummy source when gate 2 is off
    for (int b0 = 0; b0 < nb; b0 += cb) {
      const int nbc = min(cb, nb - b0);
      const int ne = nbc * H;
      const int64_t g0 = (int64_t)(off + b0) * H;
      for (int e0 = 0; e0 < ne; e0 += kEpt * (int)blockDim.x) {
        bool kk[kEpt];
        if (p.mask_in) {
          uint8_t mv[kEpt];
#pragma unroll
          for (int u = 0; u < kEpt; ++u) {
            const int e = min(e0 + u * (int)blockDim.x + t, ne - 1);
            const int mh = p.mask_in_heads;
            const int64_t ge = g0 + e;
            mv[u] = p.mask_in[mh == 1 ? (ge / H) : ge];
          }
#pragma unroll
          for (int u = 0; u < kEpt; ++u) kk[u] = mv[u] != 0;
        } else {
          float tv[kEpt], zv[kEpt];
#pragma unroll
          for (int u = 0; u < kEpt; ++u) {
            const int e = min(e0 + u * (int)blockDim.x + t, ne - 1);
            tv[u] = p.tau_max[g0 + e];
            zv[u] = zsrc[g0 + e];
          }
          for (int part = 1; part < p.tau_parts; ++part) {
            const float* tp = p.tau_max + (int64_t)part * p.total_blocks * H + g0;
            float pv[kEpt];
#pragma unroll
            for (int u = 0; u < kEpt; ++u) pv[u] = tp[min(e0 + u * (int)blockDim.x + t, ne - 1)];
#pragma unroll
            for (int u = 0; u < kEpt; ++u) tv[u] = nanmax(tv[u], pv[u]);
          }
#pragma unroll
          for (int u = 0; u < kEpt; ++u) kk[u] = (tv[u] >= tau) & ((p.zeta == nullptr) | (zv[u] <= zmax));
        }
#pragma unroll
        for (int u = 0; u < kEpt; ++u) {
          const int e = e0 + u * (int)blockDim.x + t;
          if (e < ne) {
            s_flag[e] = kk[u] ? 1 : 0;
            if (p.mask_out) p.mask_out[g0 + e] = kk[u] ? 1 : 0;
          }
        }
      }
      __syncthreads();
      bool a = false;
      if (t < nbc) {
        for (int h = 0; h < H; ++h) a |= s_flag[t * H + h] != 0;
        if (act_in_lds) s_act[b0 + t] = a ? 1 : 0;
        if (p.active_out) p.active_out[off + b0 + t] = a ? 1 : 0;
      }
      int tot;
      block_scan_bool(a, s_cnt, tot);  // its barriers also retire s_flag
      n += tot;
    }
  }

  // Pass 2: scatter the active-first stable permutation.
  if (p.indices) {
    int run_act = 0, run_in = 0;
    for (int base = 0; base < nb; base += blockDim.x) {
      const int j = base + t;
      bool a = false;
      if (j < nb) a = act_in_lds ? (s_act[j] != 0) : keep_any(p, off + j, tau, zmax);
      int tot;
      const int ex = block_scan_bool(a, s_cnt, tot);
      if (j < nb) {
        const int pos = a ? (run_act + ex) : (n + run_in + (t - ex));
        p.indices[off + pos] = j;
      }
      const int valid = min((int)blockDim.x, nb - base);
      run_act += tot;
      run_in += valid - tot;
    }
    if (t == 0 && p.num_active) p.num_active[seg] = n;
  }

  if (p.head_indices) {
    for (int h = 0; h < H; ++h) {
      int* out = p.head_indices + (int64_t)h * p.total_blocks + off;
      int nh = stable_partition(
          nb, out, [&](int j) { return keep_one(p, off + j, h, tau, zmax); }, s_cnt);
      bool uniform = false;
      if (nh == 0 && p.empty_head_all) {
        for (int j = t; j < nb; j += blockDim.x) out[j] = j;
        nh = nb;
        uniform = true;
      }
      if (t == 0) {
        p.head_num_active[seg * H + h] = nh;
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
