// Shared device helpers for the OrthoCache gfx950 kernels.
//
// Element types: fp32, bf16 and fp16 inputs are loaded 16 bytes per lane
// (global_load_dwordx4) and widened to fp32 in registers; all arithmetic on
// the path is fp32.
#pragma once

#include <hip/hip_runtime.h>
#include <hip/hip_fp16.h>
#include <stdint.h>

namespace oc {

constexpr int kBlock = 512;          // tokens per KV block (the FWHT length)
constexpr int kWave = 64;            // CDNA wavefront width
constexpr float kSqrt512 = 22.627416997969522f;  // fp32 rounding of sqrt(512)

enum DType : int { kF32 = 0, kBF16 = 1, kF16 = 2 };

__host__ __device__ constexpr int dtype_size(int dt) { return dt == kF32 ? 4 : 2; }

// ---------------------------------------------------------------- conversions
__device__ __forceinline__ float bf16_lo(uint32_t w) { return __uint_as_float(w << 16); }
__device__ __forceinline__ float bf16_hi(uint32_t w) { return __uint_as_float(w & 0xffff0000u); }

__device__ __forceinline__ uint32_t f32_to_bf16_bits(float f) {
  uint32_t u = __float_as_uint(f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return 0x7fc0u;  // quiet NaN
  u += 0x7fffu + ((u >> 16) & 1u);                       // round to nearest even
  return u >> 16;
}

__device__ __forceinline__ float f16_bits_to_f32(uint32_t h) {
  return __half2float(__ushort_as_half(static_cast<unsigned short>(h & 0xffffu)));
}

__device__ __forceinline__ uint32_t f32_to_f16_bits(float f) {
  return __half_as_ushort(__float2half_rn(f));
}

// Element type traits: VEC elements per 16-byte lane load.
template <int DT> struct Elt;
// get(w, c): element c of a 16-byte word, widened to fp32 (c is a
// compile-time constant after unrolling).
__device__ __forceinline__ uint32_t word_of(const uint4& w, int i) {
  return i == 0 ? w.x : i == 1 ? w.y : i == 2 ? w.z : w.w;
}
template <> struct Elt<kF32> {
  static constexpr int VEC = 4;
  __device__ __forceinline__ static float get(const uint4& w, int c) { return __uint_as_float(word_of(w, c)); }
  __device__ __forceinline__ static void unpack(const uint4& w, float* o) {
    o[0] = __uint_as_float(w.x); o[1] = __uint_as_float(w.y);
    o[2] = __uint_as_float(w.z); o[3] = __uint_as_float(w.w);
  }
  __device__ __forceinline__ static float load1(const void* p, int64_t i) {
    return reinterpret_cast<const float*>(p)[i];
  }
  __device__ __forceinline__ static void store1(void* p, int64_t i, float v) {
    reinterpret_cast<float*>(p)[i] = v;
  }
};
template <> struct Elt<kBF16> {
  static constexpr int VEC = 8;
  __device__ __forceinline__ static float get(const uint4& w, int c) {
    return (c & 1) ? bf16_hi(word_of(w, c / 2)) : bf16_lo(word_of(w, c / 2));
  }
  __device__ __forceinline__ static void unpack(const uint4& w, float* o) {
    o[0] = bf16_lo(w.x); o[1] = bf16_hi(w.x); o[2] = bf16_lo(w.y); o[3] = bf16_hi(w.y);
    o[4] = bf16_lo(w.z); o[5] = bf16_hi(w.z); o[6] = bf16_lo(w.w); o[7] = bf16_hi(w.w);
  }
  __device__ __forceinline__ static float load1(const void* p, int64_t i) {
    return __uint_as_float(static_cast<uint32_t>(reinterpret_cast<const uint16_t*>(p)[i]) << 16);
  }
  __device__ __forceinline__ static void store1(void* p, int64_t i, float v) {
    reinterpret_cast<uint16_t*>(p)[i] = static_cast<uint16_t>(f32_to_bf16_bits(v));
  }
};
template <> struct Elt<kF16> {
  static constexpr int VEC = 8;
  __device__ __forceinline__ static float get(const uint4& w, int c) {
    return f16_bits_to_f32(word_of(w, c / 2) >> (16 * (c & 1)));
  }
  __device__ __forceinline__ static void unpack(const uint4& w, float* o) {
    o[0] = f16_bits_to_f32(w.x); o[1] = f16_bits_to_f32(w.x >> 16);
    o[2] = f16_bits_to_f32(w.y); o[3] = f16_bits_to_f32(w.y >> 16);
    o[4] = f16_bits_to_f32(w.z); o[5] = f16_bits_to_f32(w.z >> 16);
    o[6] = f16_bits_to_f32(w.w); o[7] = f16_bits_to_f32(w.w >> 16);
  }
  __device__ __forceinline__ static float load1(const void* p, int64_t i) {
    return f16_bits_to_f32(reinterpret_cast<const uint16_t*>(p)[i]);
  }
  __device__ __forceinline__ static void store1(void* p, int64_t i, float v) {
    reinterpret_cast<uint16_t*>(p)[i] = static_cast<uint16_t>(f32_to_f16_bits(v));
  }
};

__device__ __forceinline__ float load_elt(int dt, const void* p, int64_t i) {
  return dt == kF32 ? Elt<kF32>::load1(p, i) : (dt == kBF16 ? Elt<kBF16>::load1(p, i)
                                                            : Elt<kF16>::load1(p, i));
}
__device__ __forceinline__ void store_elt(int dt, void* p, int64_t i, float v) {
  if (dt == kF32) Elt<kF32>::store1(p, i, v);
  else if (dt == kBF16) Elt<kBF16>::store1(p, i, v);
  else Elt<kF16>::store1(p, i, v);
}

// acc + a.lo * b.lo + a.hi * b.hi for two packed 16-bit floats per operand
// (v_dot2c_f32_bf16 / v_dot2c_f32_f16): the products are exact in fp32 and
// accumulate in fp32.
template <int DT>
__device__ __forceinline__ float dot2_acc(uint32_t a, uint32_t b, float acc) {
  static_assert(DT == kBF16 || DT == kF16, "16-bit types only");
  if constexpr (DT == kBF16) {
    typedef __bf16 v2bf __attribute__((ext_vector_type(2)));
    return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(v2bf, a), __builtin_bit_cast(v2bf, b), acc, false);
  } else {
    typedef _Float16 v2h __attribute__((ext_vector_type(2)));
    return __builtin_amdgcn_fdot2(__builtin_bit_cast(v2h, a), __builtin_bit_cast(v2h, b), acc, false);
  }
}

// Load of data that no lane writes while the kernel runs (lists, counts,
// segment tables), through the constant address space: with a wave-uniform
// address this is a scalar load, which waits on its own counter instead of
// behind the vector loads in flight.
template <typename T>
__device__ __forceinline__ T ld_const(const T* p) {
  typedef const __attribute__((address_space(4))) T ConstT;
  return *(ConstT*)(p);
}

// 16-byte global load (the caller guarantees 16-byte alignment).
__device__ __forceinline__ uint4 ld16(const void* p) {
  return *reinterpret_cast<const uint4*>(p);
}

// 16-byte non-temporal load for data streamed once (keys, retained K/V): the
// line is not kept in the caches, which measurably raises streaming HBM
// bandwidth on gfx950.
__device__ __forceinline__ uint4 ld16_nt(const void* p) {
  typedef unsigned int v4u __attribute__((ext_vector_type(4)));
  const v4u w = __builtin_nontemporal_load(reinterpret_cast<const v4u*>(p));
  return make_uint4(w.x, w.y, w.z, w.w);
}

// 16-byte non-temporal store for data the kernel writes once and another
// launch reads (the scoring pass's logits): the line is not kept dirty in the
// writer's L2.  C2 decode layer 107.0-107.8 -> 105.5-106.0 us.
__device__ __forceinline__ void st16_nt(void* p, float4 v) {
  typedef float v4f __attribute__((ext_vector_type(4)));
  const v4f w = {v.x, v.y, v.z, v.w};
  __builtin_nontemporal_store(w, reinterpret_cast<v4f*>(p));
}

// 4-byte form, for the prefill kernel's transposed split partials (C4 chunk
// 139.2 -> 138.7 us in a same-box A/B; the decode partials measured slower
// this way).
__device__ __forceinline__ void st4_nt(float* p, float v) { __builtin_nontemporal_store(v, p); }

// Workgroup barrier that orders LDS accesses only: s_waitcnt lgkmcnt(0) +
// s_barrier, without waiting for the vector memory loads in flight.
__device__ __forceinline__ void lds_barrier() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

// -------------------------------------------------------------- reductions
// jnp.max semantics: NaN in either operand propagates.
__device__ __forceinline__ float nanmax(float a, float b) { return (a > b || a != a) ? a : b; }

template <int WIDTH>
__device__ __forceinline__ float group_sum(float v) {
#pragma unroll
  for (int o = WIDTH / 2; o > 0; o >>= 1) v += __shfl_xor(v, o, WIDTH);
  return v;
}

__device__ __forceinline__ float wave_sum(float v) { return group_sum<kWave>(v); }

// Value of lane (lane ^ B) for B in {1, 2, 4, 8, 16}, without the LDS
// crossbar: DPP quad_perm [1,0,3,2] / [2,3,0,1], ds_swizzle bit-mask xor 4
// and 16 (within 32 lanes), DPP row_ror:8 (xor 8 within a 16-lane row).
// Lane mappings pinned on gfx950 by an in-bounds probe.
template <int B>
__device__ __forceinline__ float lane_xor(float v) {
  const int x = __float_as_int(v);
  if constexpr (B == 1) return __int_as_float(__builtin_amdgcn_update_dpp(0, x, 0xB1, 0xF, 0xF, false));
  else if constexpr (B == 2) return __int_as_float(__builtin_amdgcn_update_dpp(0, x, 0x4E, 0xF, 0xF, false));
  else if constexpr (B == 4) return __int_as_float(__builtin_amdgcn_ds_swizzle(x, 0x101F));
  else if constexpr (B == 8) return __int_as_float(__builtin_amdgcn_update_dpp(0, x, 0x128, 0xF, 0xF, false));
  else if constexpr (B == 16) return __int_as_float(__builtin_amdgcn_ds_swizzle(x, 0x401F));
  else return __shfl_xor(v, B, kWave);
}

// One pair step of B = 16 or 32 with v_permlane{16,32}_swap: lanes whose bit
// B is clear get x + x(lane ^ B), the others y(lane ^ B) + y.  That is the
// halving-butterfly step for (x, y) = (v[i], v[i + H]) with no selects, and
// the plain exchange-and-add for x = y.
template <int B>
__device__ __forceinline__ float swap_add(float x, float y) {
  static_assert(B == 16 || B == 32, "row swaps pair 16- or 32-lane rows");
  if constexpr (B == 16) {
    const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(y), false, false);
    return __uint_as_float(r[0]) + __uint_as_float(r[1]);
  } else {
    const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(y), false, false);
    return __uint_as_float(r[0]) + __uint_as_float(r[1]);
  }
}

// Halving butterfly: sums V per-lane values over groups of LPR lanes.  With
// V >= LPR, lane l ends with the full sums of value indices
// [l*V/LPR, (l+1)*V/LPR) in v[0..V/LPR); with V < LPR, v[0] of lane l is the
// sum of index l / (LPR/V).  V - 1 exchanges for V values instead of
// V log2(LPR).  Instantiate as Butterfly<V, V, LPR / 2, LPR>.
template <int V, int CNT, int B, int LPR>
struct Butterfly {
  __device__ __forceinline__ static void run(float (&v)[V], int lane) {
    if constexpr (B >= 1) {
      if constexpr (CNT > 1) {
        constexpr int H = CNT / 2;
        if constexpr (B >= 16) {
#pragma unroll
          for (int i = 0; i < H; ++i) v[i] = swap_add<B>(v[i], v[i + H]);
        } else {
          const bool upper = (lane & B) != 0;
#pragma unroll
          for (int i = 0; i < H; ++i) {
            const float send = upper ? v[i] : v[i + H];
            const float keep = upper ? v[i + H] : v[i];
            v[i] = keep + lane_xor<B>(send);
          }
        }
        Butterfly<V, H, B / 2, LPR>::run(v, lane);
      } else {
        if constexpr (B >= 16) v[0] = swap_add<B>(v[0], v[0]);
        else v[0] += lane_xor<B>(v[0]);
        Butterfly<V, 1, B / 2, LPR>::run(v, lane);
      }
    }
  }
};

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int o = kWave / 2; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, kWave));
  return v;
}

// Sum N values over the whole workgroup; every thread receives the totals.
// lds must hold N * (blockDim.x / 64) floats.  Contains two barriers.
template <int N>
__device__ __forceinline__ void block_sum(float (&v)[N], float* lds) {
  const int lane = threadIdx.x & (kWave - 1);
  const int wave = threadIdx.x / kWave;
  const int nwaves = (blockDim.x + kWave - 1) / kWave;
#pragma unroll
  for (int i = 0; i < N; ++i) v[i] = wave_sum(v[i]);
  if (lane == 0) {
#pragma unroll
    for (int i = 0; i < N; ++i) lds[i * nwaves + wave] = v[i];
  }
  __syncthreads();
#pragma unroll
  for (int i = 0; i < N; ++i) {
    float s = 0.f;
    for (int w = 0; w < nwaves; ++w) s += lds[i * nwaves + w];
    v[i] = s;
  }
  __syncthreads();
}

}  // namespace oc
