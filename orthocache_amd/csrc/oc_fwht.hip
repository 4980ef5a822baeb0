// Standalone 512-point fast Walsh-Hadamard transform, natural order, scaled
// by 1/sqrt(512): replaces fwht_512 (src/orthocache/fwht.py:4-65) and the
// blocked form _run_fwht_on_blocks (src/orthocache/spectral_energy.py:38-66).
//
// The transform runs along rows (stride row_stride elements) of a batch of
// 512 x n_cols tiles; columns are contiguous.  A workgroup of 256 threads
// takes a 512 x 32 column tile:
//   phase 1: thread (column c, row group k = 0..7) loads rows 64k + l,
//            l = 0..63, and runs the six butterfly stages over l (bits 0-5)
//            in registers;
//   phase 2: after an LDS transpose, thread (column c, l-group) runs the three
//            stages over k (bits 6-8) for eight values of l and stores.
// Arithmetic is fp32 whatever the input/output storage type.
#include "oc_kernels.h"

namespace oc {

constexpr int kFwhtCols = 32;

__global__ __launch_bounds__(256) void fwht512_kernel(FwhtParams p) {
  __shared__ float tile[kBlock * kFwhtCols];
  const int64_t ctiles = (p.n_cols + kFwhtCols - 1) / kFwhtCols;
  const int64_t bt = blockIdx.x / ctiles;
  const int64_t ct = blockIdx.x - bt * ctiles;
  const int t = threadIdx.x;
  const int c = t % kFwhtCols;
  const int grp = t / kFwhtCols;  // 0..7
  const int64_t col = ct * kFwhtCols + c;
  const bool live = col < p.n_cols;
  const int64_t xb = bt * p.x_batch_stride + col;
  const int64_t yb = bt * p.y_batch_stride + col;

  float v[64];
#pragma unroll
  for (int l = 0; l < 64; ++l)
    v[l] = live ? load_elt(p.x_dtype, p.x, xb + (int64_t)(64 * grp + l) * p.x_row_stride) : 0.f;
#pragma unroll
  for (int h = 1; h < 64; h <<= 1) {
#pragma unroll
    for (int i = 0; i < 64; i += 2 * h) {
#pragma unroll
      for (int j = i; j < i + h; ++j) {
        const float a = v[j], b = v[j + h];
        v[j] = a + b;
        v[j + h] = a - b;
      }
    }
  }
#pragma unroll
  for (int l = 0; l < 64; ++l) tile[(64 * grp + l) * kFwhtCols + c] = v[l];
  __syncthreads();

  const int lg = grp;  // l in [8*lg, 8*lg + 8)
#pragma unroll
  for (int li = 0; li < 8; ++li) {
    const int l = 8 * lg + li;
    float w[8];
#pragma unroll
    for (int k = 0; k < 8; ++k) w[k] = tile[(64 * k + l) * kFwhtCols + c];
#pragma unroll
    for (int h = 1; h < 8; h <<= 1) {
#pragma unroll
      for (int i = 0; i < 8; i += 2 * h) {
#pragma unroll
        for (int j = i; j < i + h; ++j) {
          const float a = w[j], b = w[j + h];
          w[j] = a + b;
          w[j + h] = a - b;
        }
      }
    }
    if (live) {
#pragma unroll
      for (int k = 0; k < 8; ++k)
        store_elt(p.y_dtype, p.y, yb + (int64_t)(64 * k + l) * p.y_row_stride, w[k] / kSqrt512);
    }
  }
}

// Band energy over a materialised spectrum (nb, 512, H, D) fp32:
// out[b, h] = sum_{s in [s0, s1)} sum_d spec[b, s, h, d]^2.
// Used for band boundaries other than the default ones
// (spectral_energy.py:69-106 takes them as arguments).
__global__ __launch_bounds__(256) void band_energy_kernel(BandParams p) {
  __shared__ float s_red[8];
  const int b = blockIdx.x / p.num_heads, h = blockIdx.x - b * p.num_heads;
  const int n = (p.s1 - p.s0) * p.head_dim;
  float acc = 0.f;
  for (int e = threadIdx.x; e < n; e += blockDim.x) {
    const int s = p.s0 + e / p.head_dim, d = e % p.head_dim;
    const float v = p.spec[(((int64_t)b * kBlock + s) * p.num_heads + h) * p.head_dim + d];
    acc = fmaf(v, v, acc);
  }
  float v1[1] = {acc};
  block_sum<1>(v1, s_red);
  if (threadIdx.x == 0) p.out[blockIdx.x] = v1[0];
}

hipError_t launch_fwht(const FwhtParams& p, hipStream_t s) {
  const int64_t ctiles = (p.n_cols + kFwhtCols - 1) / kFwhtCols;
  const int64_t grid = ctiles * p.n_batch;
  if (grid == 0) return hipSuccess;
  hipLaunchKernelGGL(fwht512_kernel, dim3((unsigned)grid), dim3(256), 0, s, p);
  return hipGetLastError();
}

hipError_t launch_band_energy(const BandParams& p, hipStream_t s) {
  if (p.num_blocks * p.num_heads == 0) return hipSuccess;
  hipLaunchKernelGGL(band_energy_kernel, dim3(p.num_blocks * p.num_heads), dim3(256), 0, s, p);
  return hipGetLastError();
}

}  // namespace oc
