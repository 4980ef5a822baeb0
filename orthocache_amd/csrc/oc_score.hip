// Block scoring: spectral bands, zeta, block mean and the query-aware bound.
//
// Replaces the reference's compute_spectral_bands / compute_spectral_decay_ratio
// / compute_query_aware_bounds / compute_query_aware_mask
// (src/orthocache/spectral_energy.py:69-196), which materialise the full
// 512-point FWHT of every (block, head, dim) column.  The bands are ranges of
// natural (Hadamard) coefficient indices: DC = {0}, low = [1,64),
// mid = [64,256), high = [256,512), i.e. cosets of the top three index bits.
// By Parseval, the energy of a coset only needs the butterflies over token
// bits 6, 7 and 8.  Write a token index as i = 64*k + l (k in 0..7, l in 0..63)
// and, per column and per l, x_k = K[64k + l]:
//   E_high = 1/2 * sum_l sum_{k<4} (x_k - x_{k+4})^2            (index bit 8 set)
//   u_k    = x_k + x_{k+4},  y = WHT4(u)
//   E_mid  = 1/8 * sum_l (y1^2 + y2^2 + y3^2)                    (bits 6/7 set, 8 clear)
//          = 1/8 * sum_l (2 a1^2 + 2 a3^2 + y2^2), with a1 = u0 - u1, a3 = u2 - u3,
//            since y1^2 + y3^2 = (a1 + a3)^2 + (a1 - a3)^2
//   E_low  = 1/8 * sum_l (y0_l - mean_l y0)^2                    (coset 0 minus DC)
//   DC     = sum_l y0_l / sqrt(512),  kbar = DC / sqrt(512)
// so one pass over the keys, ~4 VALU ops per element, gives every score the
// reference derives from the full spectrum.  E_low is formed as a centred sum
// of squares (shifted sums per thread, Chan merge across threads), so a large
// block mean does not cancel it away.
//
// One workgroup (256 threads) scores one (block, kv head) tile of 512 x D.
// Lanes are laid out LPR per token row (16-byte loads along D, coalesced);
// NSLOT = 256/LPR row slots each walk 64/NSLOT values of l, loading the eight
// rows 64k + l together.
#include "oc_kernels.h"

namespace oc {

template <int DT, int LPR>
__device__ __forceinline__ void load_rows(const char* base, int64_t row_bytes, int l, uint4 (&r)[8]) {
#pragma unroll
  for (int k = 0; k < 8; ++k) r[k] = ld16_nt(base + (int64_t)(64 * k + l) * row_bytes);
}

constexpr int kMaxSegLds = 4096;  // segments whose offsets are staged in LDS

template <int DT, int LPR, int QDT>
__global__ __launch_bounds__(256) void score_kernel(ScoreParams p) {
  using E = Elt<DT>;
  using EQ = Elt<QDT>;
  constexpr int VEC = E::VEC;
  constexpr int D = LPR * VEC;
  constexpr int NSLOT = 256 / LPR;
  constexpr int NLO = 64 / NSLOT;
  static_assert(NLO >= 2 && (NLO % 2) == 0, "unsupported lane layout");
  constexpr int ESZ = (DT == kF32) ? 4 : 2;

  constexpr int NI = (D + 255) / 256;  // head_dim columns per thread in the epilogue
  __shared__ float s_mean[NSLOT * D];
  __shared__ float s_m2[NSLOT * D];
  __shared__ float s_red[64];
  __shared__ int s_cu[kMaxSegLds + 1];

  const int tile = blockIdx.x;
  const int H = p.num_kv_heads;
  const int gb = tile / H;
  const int h = tile - gb * H;
  const int t = threadIdx.x;
  const int cc = t % LPR;
  const int slot = t / LPR;

  const int64_t row_bytes = p.k_tok_stride * ESZ;
  const char* base = reinterpret_cast<const char*>(p.k) +
                     ((int64_t)gb * kBlock * p.k_tok_stride + (int64_t)h * p.k_head_stride +
                      (int64_t)cc * VEC) * ESZ;

  // Query-aware bound inputs, requested before the key stream so their
  // latency overlaps it: the segment table (ragged batches) goes to LDS, the
  // first four queries' values of this thread's columns go to registers
  // (one segment; a ragged batch needs the segment id first).
  const bool want_bound = p.q != nullptr && p.tau_max != nullptr;
  const int nq = p.sq * p.group;
  const bool need_seg = p.cu_blocks != nullptr && want_bound;
  if (need_seg) {
    for (int i = t; i <= p.num_segments; i += 256) s_cu[i] = p.cu_blocks[i];
  }
  float qpre[4][NI];
  const bool prefetch = want_bound && p.cu_blocks == nullptr && nq > 0;
  if (prefetch) {
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int qi = min(u, nq - 1);
      const int st = qi / p.group, g = qi - st * p.group;
      const int64_t qoff = (int64_t)st * p.q_tok_stride + (int64_t)(h * p.group + g) * p.q_head_stride;
#pragma unroll
      for (int i = 0; i < NI; ++i) qpre[u][i] = EQ::load1(p.q, qoff + min(t + 256 * i, D - 1));
    }
  }

  float acc_hi[VEC], acc_mid[VEC], acc_mid2[VEC], piv[VEC], ssum[VEC], ssq[VEC];
#pragma unroll
  for (int c = 0; c < VEC; ++c) { acc_hi[c] = 0.f; acc_mid[c] = 0.f; acc_mid2[c] = 0.f; ssum[c] = 0.f; ssq[c] = 0.f; piv[c] = 0.f; }

  auto consume = [&](const uint4 (&r)[8], bool first) {
    float x[8][VEC];
#pragma unroll
    for (int k = 0; k < 8; ++k) E::unpack(r[k], x[k]);
#pragma unroll
    for (int c = 0; c < VEC; ++c) {
      const float d0 = x[0][c] - x[4][c], d1 = x[1][c] - x[5][c];
      const float d2 = x[2][c] - x[6][c], d3 = x[3][c] - x[7][c];
      float ah = acc_hi[c];
      ah = fmaf(d0, d0, ah); ah = fmaf(d1, d1, ah); ah = fmaf(d2, d2, ah); ah = fmaf(d3, d3, ah);
      acc_hi[c] = ah;
      const float u0 = x[0][c] + x[4][c], u1 = x[1][c] + x[5][c];
      const float u2 = x[2][c] + x[6][c], u3 = x[3][c] + x[7][c];
      const float a0 = u0 + u1, a1 = u0 - u1, a2 = u2 + u3, a3 = u2 - u3;
      const float y0 = a0 + a2, y2 = a0 - a2;
      float am = acc_mid[c], am2 = acc_mid2[c];
      am2 = fmaf(a1, a1, am2); am2 = fmaf(a3, a3, am2); am = fmaf(y2, y2, am);
      acc_mid[c] = am; acc_mid2[c] = am2;
      if (first) {
        piv[c] = y0;
      } else {
        const float dv = y0 - piv[c];
        ssum[c] += dv;
        ssq[c] = fmaf(dv, dv, ssq[c]);
      }
    }
  };

  uint4 ra[8], rb[8];
  load_rows<DT, LPR>(base, row_bytes, slot, ra);
#pragma unroll
  for (int j = 0; j < NLO; j += 2) {
    load_rows<DT, LPR>(base, row_bytes, slot + NSLOT * (j + 1), rb);
    consume(ra, j == 0);
    if (j + 2 < NLO) load_rows<DT, LPR>(base, row_bytes, slot + NSLOT * (j + 2), ra);
    consume(rb, false);
  }

  float hi = 0.f, mid = 0.f;
#pragma unroll
  for (int c = 0; c < VEC; ++c) {
    hi += acc_hi[c];
    mid += acc_mid[c] + 2.f * acc_mid2[c];
    const float mean_t = piv[c] + ssum[c] * (1.f / NLO);
    // Clamp rounding below zero without dropping NaN (fmaxf would).
    const float m2_raw = ssq[c] - ssum[c] * ssum[c] * (1.f / NLO);
    const float m2_t = m2_raw < 0.f ? 0.f : m2_raw;
    s_mean[slot * D + cc * VEC + c] = mean_t;
    s_m2[slot * D + cc * VEC + c] = m2_t;
  }
  __syncthreads();

  // Per column: merge the NSLOT partial (mean, M2) pairs (equal counts NLO).
  float elow = 0.f;
  float kbar_r[NI];
#pragma unroll
  for (int i = 0; i < NI; ++i) {
    const int d = t + 256 * i;
    kbar_r[i] = 0.f;
    if (d < D) {
      float m = 0.f;
#pragma unroll
      for (int s = 0; s < NSLOT; ++s) m += s_mean[s * D + d];
      m *= (1.f / NSLOT);
      float m2 = 0.f;
#pragma unroll
      for (int s = 0; s < NSLOT; ++s) {
        const float dm = s_mean[s * D + d] - m;
        m2 += s_m2[s * D + d] + (float)NLO * dm * dm;
      }
      elow += m2;
      const float dcv = (64.f * m) / kSqrt512;  // sum over l of y0, over sqrt(512)
      if (p.dc) p.dc[(int64_t)tile * D + d] = dcv;
      kbar_r[i] = dcv / kSqrt512;                // spectral_energy.py:166
    }
  }

  float tot[3] = {hi, mid, elow};
  block_sum<3>(tot, s_red);
  const float e_high = 0.5f * tot[0];
  const float e_mid = 0.125f * tot[1];
  const float e_low = 0.125f * tot[2];
  const float e_ac = e_low + e_mid + e_high;
  if (t == 0) {
    if (p.e_low) p.e_low[tile] = e_low;
    if (p.e_mid) p.e_mid[tile] = e_mid;
    if (p.e_high) p.e_high[tile] = e_high;
    if (p.e_ac) p.e_ac[tile] = e_ac;
    if (p.zeta) p.zeta[tile] = e_high / (e_low + 1e-6f);  // spectral_energy.py:138
  }

  // Inline query-aware bound: tau_j = q.kbar/sqrt(d) + ||q|| sqrt(E_AC)/sqrt(d),
  // max over the segment's queries of every query head sharing kv head h.
  int seg = 0;
  if (need_seg) {
    // s_cu was filled before the key stream; block_sum's barriers have
    // made it visible.  Binary search for the segment holding block gb.
    int lo = 0, hi = p.num_segments - 1;
    while (lo < hi) {
      const int mid = (lo + hi + 1) >> 1;
      if (s_cu[mid] <= gb) lo = mid; else hi = mid - 1;
    }
    seg = lo;
  }
  if (want_bound) {
    const float sqrt_d = sqrtf((float)D);
    const float sqrt_eac = sqrtf(e_ac);
    float best = -INFINITY;
    for (int q0 = 0; q0 < nq; q0 += 4) {
      float qv[4][NI];
      if (prefetch && q0 == 0) {
#pragma unroll
        for (int u = 0; u < 4; ++u)
#pragma unroll
          for (int i = 0; i < NI; ++i) qv[u][i] = qpre[u][i];
      } else {
#pragma unroll
        for (int u = 0; u < 4; ++u) {
          const int qi = min(q0 + u, nq - 1);
          const int st = qi / p.group, g = qi - st * p.group;
          const int64_t qoff = (int64_t)seg * p.q_seg_stride + (int64_t)st * p.q_tok_stride +
                               (int64_t)(h * p.group + g) * p.q_head_stride;
#pragma unroll
          for (int i = 0; i < NI; ++i) qv[u][i] = EQ::load1(p.q, qoff + min(t + 256 * i, D - 1));
        }
      }
      float part[8];
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        float a = 0.f, b = 0.f;
#pragma unroll
        for (int i = 0; i < NI; ++i) {
          const float v = (t + 256 * i < D) ? qv[u][i] : 0.f;
          a = fmaf(v, kbar_r[i], a);
          b = fmaf(v, v, b);
        }
        part[2 * u] = a;
        part[2 * u + 1] = b;
      }
      block_sum<8>(part, s_red);
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        if (q0 + u < nq) {
          const float align = part[2 * u] / sqrt_d;
          const float resid = (sqrtf(part[2 * u + 1]) * sqrt_eac) / sqrt_d;
          best = nanmax(align + resid, best);
        }
      }
    }
    if (t == 0) p.tau_max[tile] = best;
  }
}

// Query-aware bound for many queries (prefill): one workgroup per
// (query tile of 32, block tile of 8, kv head).  Needs kbar (from dc) and
// E_AC from score_kernel.  Writes the full bound tensor (Sq*G, nb, Hkv) and/or
// the per-query-tile NaN-propagating max (ntiles, nb, Hkv).
constexpr int kBoundQT = 32;
constexpr int kBoundBT = 8;

__global__ __launch_bounds__(256) void bound_kernel(BoundParams p) {
  extern __shared__ float smem[];
  const int D = p.head_dim;
  const int DP = D + 1;
  float* s_q = smem;                       // kBoundQT x DP
  float* s_k = smem + kBoundQT * DP;       // kBoundBT x DP
  const int nq = p.sq * p.group;
  const int nqt = (nq + kBoundQT - 1) / kBoundQT;
  const int nbt = (p.num_blocks + kBoundBT - 1) / kBoundBT;
  int id = blockIdx.x;
  const int h = id % p.num_kv_heads; id /= p.num_kv_heads;
  const int bt = id % nbt;
  const int qt = id / nbt;
  if (qt >= nqt) return;
  const int t = threadIdx.x;
  for (int e = t; e < kBoundQT * D; e += blockDim.x) {
    const int r = e / D, d = e - r * D;
    const int qi = qt * kBoundQT + r;
    float v = 0.f;
    if (qi < nq) {
      const int st = qi / p.group, g = qi - st * p.group;
      v = load_elt(p.q_dtype, p.q, (int64_t)st * p.q_tok_stride + (int64_t)(h * p.group + g) * p.q_head_stride + d);
    }
    s_q[r * DP + d] = v;
  }
  for (int e = t; e < kBoundBT * D; e += blockDim.x) {
    const int r = e / D, d = e - r * D;
    const int b = bt * kBoundBT + r;
    s_k[r * DP + d] = (b < p.num_blocks) ? p.dc[((int64_t)b * p.num_kv_heads + h) * D + d] / kSqrt512 : 0.f;
  }
  __syncthreads();
  const int ql = t % kBoundQT;
  const int bl = t / kBoundQT;   // 0..7
  const int qi = qt * kBoundQT + ql;
  const int b = bt * kBoundBT + bl;
  float dot = 0.f, qq = 0.f;
  for (int d = 0; d < D; ++d) {
    const float qv = s_q[ql * DP + d];
    dot = fmaf(qv, s_k[bl * DP + d], dot);
    qq = fmaf(qv, qv, qq);
  }
  const bool valid = (qi < nq) && (b < p.num_blocks);
  float bound = -INFINITY;
  if (valid) {
    const float sqrt_d = sqrtf((float)D);
    const float eac = p.e_ac[(int64_t)b * p.num_kv_heads + h];
    bound = dot / sqrt_d + (sqrtf(qq) * sqrtf(eac)) / sqrt_d;
    if (p.bounds) p.bounds[((int64_t)qi * p.num_blocks + b) * p.num_kv_heads + h] = bound;
  }
  if (p.tau_part) {
    // NaN-propagating max over the 32 queries of this tile (lanes ql share bl
    // within one wave: 64 lanes = 2 block rows x 32 queries).
    float m = bound;
#pragma unroll
    for (int o = kBoundQT / 2; o > 0; o >>= 1) m = nanmax(m, __shfl_xor(m, o, kBoundQT));
    if (ql == 0 && b < p.num_blocks)
      p.tau_part[((int64_t)qt * p.num_blocks + b) * p.num_kv_heads + h] = m;
  }
}

// Spatial energy sum k^2 per (block, head) for any block size
// (spectral_energy.py:21-35).  One workgroup per (block, head).
__global__ __launch_bounds__(256) void block_energy_kernel(EnergyParams p) {
  __shared__ float s_red[8];
  const int tile = blockIdx.x;
  const int b = tile / p.num_kv_heads, h = tile - b * p.num_kv_heads;
  const int n = p.block_size * p.head_dim;
  float acc = 0.f;
  for (int e = threadIdx.x; e < n; e += blockDim.x) {
    const int r = e / p.head_dim, d = e - r * p.head_dim;
    const float v = load_elt(p.k_dtype, p.k, ((int64_t)b * p.block_size + r) * p.k_tok_stride +
                                              (int64_t)h * p.k_head_stride + d);
    acc = fmaf(v, v, acc);
  }
  float v1[1] = {acc};
  block_sum<1>(v1, s_red);
  if (threadIdx.x == 0) p.out[tile] = v1[0];
}

}  // namespace oc

// ---------------------------------------------------------------- launchers
namespace oc {

template <int DT, int LPR>
static hipError_t launch_score_t(const ScoreParams& p, hipStream_t s) {
  const int tiles = p.total_blocks * p.num_kv_heads;
  // Without queries the query type is irrelevant: use the key type.
  const int qdt = p.q ? p.q_dtype : DT;
  if (qdt == DT) {
    hipLaunchKernelGGL((score_kernel<DT, LPR, DT>), dim3(tiles), dim3(256), 0, s, p);
  } else if (qdt == kF32) {
    hipLaunchKernelGGL((score_kernel<DT, LPR, kF32>), dim3(tiles), dim3(256), 0, s, p);
  } else {
    return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

template <int DT>
static hipError_t launch_score_dt(const ScoreParams& p, hipStream_t s) {
  const int lpr = p.head_dim / Elt<DT>::VEC;
  switch (lpr) {
    case 8: return launch_score_t<DT, 8>(p, s);
    case 16: return launch_score_t<DT, 16>(p, s);
    case 32: return launch_score_t<DT, 32>(p, s);
    case 64: return launch_score_t<DT, 64>(p, s);
    case 128: return launch_score_t<DT, 128>(p, s);
    default: return hipErrorInvalidValue;
  }
}

// True when score_kernel has an instantiation for (dtype, head_dim).
bool score_supported(int dt, int head_dim) {
  const int vec = (dt == kF32) ? 4 : 8;
  if (head_dim % vec) return false;
  const int lpr = head_dim / vec;
  return lpr == 8 || lpr == 16 || lpr == 32 || lpr == 64 || lpr == 128;
}

hipError_t launch_score(const ScoreParams& p, hipStream_t s) {
  if (p.total_blocks == 0) return hipSuccess;
  switch (p.k_dtype) {
    case kF32: return launch_score_dt<kF32>(p, s);
    case kBF16: return launch_score_dt<kBF16>(p, s);
    case kF16: return launch_score_dt<kF16>(p, s);
    default: return hipErrorInvalidValue;
  }
}

hipError_t launch_bound(const BoundParams& p, hipStream_t s) {
  const int nq = p.sq * p.group;
  if (nq == 0 || p.num_blocks == 0) return hipSuccess;
  const int nqt = (nq + kBoundQT - 1) / kBoundQT;
  const int nbt = (p.num_blocks + kBoundBT - 1) / kBoundBT;
  const size_t lds = (size_t)(kBoundQT + kBoundBT) * (p.head_dim + 1) * sizeof(float);
  if (lds > 65536) {
    const hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(&bound_kernel),
                                             hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
    if (e != hipSuccess) return e;
  }
  hipLaunchKernelGGL(bound_kernel, dim3(nqt * nbt * p.num_kv_heads), dim3(256), lds, s, p);
  return hipGetLastError();
}

hipError_t launch_block_energy(const EnergyParams& p, hipStream_t s) {
  if (p.num_blocks == 0) return hipSuccess;
  hipLaunchKernelGGL(block_energy_kernel, dim3(p.num_blocks * p.num_kv_heads), dim3(256), 0, s, p);
  return hipGetLastError();
}

}  // namespace oc
