// Indirect block-sparse attention, prefill form (many queries per kv head),
// on the bf16/fp16 matrix cores.
//
// Same semantics as the decode form (oc_attend.hip) and the reference's
// orthocache_attention loop (src/orthocache/adaptive_attention.py:46-184):
// softmax(q.k / sqrt(d)) over the tokens of exactly the retained blocks, fp32
// softmax state, output o / l; an empty list yields zeros.  Used when a kv head
// has enough query rows (query tokens x heads of its group) that Q K^T and P V
// are dense contractions (chunked prefill).
//
// Work decomposition: a workgroup (8 waves for head_dim 128, 4 for 64; 32
// query rows per wave, so each staged K / V^T tile serves 256 or 128 rows)
// takes one query tile of a (segment, kv head) and a contiguous range of the
// list's 64-key tiles (the
// tile range is split `nsplit` ways so the grid fills the chip); it writes a
// partial (m, l, O) per row and prefill_combine_kernel merges the splits.
//
// Per wave: 32 query rows, one per lane pair (lane l and l^32 hold row l%32).
// With v_mfma_f32_32x32x16 (A 32x16, B 16x32, fp32 C 32x32):
//   S^T = K Q^T   A = K tile rows from LDS (16 B per lane), B = Q^T slice from
//                 registers (loaded once), C lane l, i -> key 8(i/4)+4(l/32)+i%4,
//                 query l%32;
//   O^T += V^T P^T  A = V^T from a transposed LDS copy, B = P^T straight from
//                 the S^T registers (converted to bf16/fp16), C -> d, query l%32.
// So every query's softmax state (m, l) and its column of O^T stay in the two
// lanes that own the query: no shuffles except one xor-32 per tile for the row
// max.  The MFMA k index of P^T / V^T is a permutation of the 16 keys of a
// slice (the keys a lane holds in S^T); the V^T copy in LDS stores keys in that
// order so the A operand is one 16-byte read.
//
// LDS: K tile [64 keys][D] and V^T tile [D][64 keys], both with 16-byte blocks
// XOR-swizzled by row so operand reads and the transposing writes spread over
// the banks.  Global loads of the next tile are issued into registers before
// the current tile's arithmetic.
#include "oc_kernels.h"

namespace oc {

namespace {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x16_t __attribute__((ext_vector_type(16)));
typedef unsigned int u32x4_t __attribute__((ext_vector_type(4)));

constexpr int kPfMaxThreads = 8 * kWave;  // largest prefill workgroup (head_dim 128)
static_assert(prefill_waves(128) * kWave == kPfMaxThreads, "workgroup size");
constexpr int kPfKeys = 64;             // keys per tile
constexpr float kLazy = 8.f;            // log2 headroom before the softmax reference moves
// (1, 1) as a packed pair of the operand type, for row sums by dot2.
template <int DT> constexpr uint32_t kOnePair = DT == kBF16 ? 0x3f803f80u : 0x3c003c00u;

template <int DT> struct Mma;
template <> struct Mma<kBF16> {
  __device__ __forceinline__ static f32x16_t run(u32x4_t a, u32x4_t b, f32x16_t c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8_t, a),
                                                   __builtin_bit_cast(bf16x8_t, b), c, 0, 0, 0);
  }
  __device__ __forceinline__ static u32x4_t pack(const float* v) {
    bf16x8_t r;
#pragma unroll
    for (int j = 0; j < 8; ++j) r[j] = (__bf16)v[j];
    return __builtin_bit_cast(u32x4_t, r);
  }
};
template <> struct Mma<kF16> {
  __device__ __forceinline__ static f32x16_t run(u32x4_t a, u32x4_t b, f32x16_t c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8_t, a),
                                                  __builtin_bit_cast(f16x8_t, b), c, 0, 0, 0);
  }
  __device__ __forceinline__ static u32x4_t pack(const float* v) {
    f16x8_t r;
#pragma unroll
    for (int j = 0; j < 8; ++j) r[j] = (_Float16)v[j];
    return __builtin_bit_cast(u32x4_t, r);
  }
};

__device__ __forceinline__ u32x4_t ld16v(const char* p) {
  return *reinterpret_cast<const u32x4_t*>(p);
}

// Position of key k (0..63) of a tile in the V^T rows: the 8 keys that lane
// half hf supplies for MFMA k-slice s of S^T tile t are contiguous.
__host__ __device__ constexpr int vt_pos(int k) {
  const int t = k >> 5, s = (k >> 4) & 1, r = k & 15;
  const int hf = (r >> 2) & 1, j = ((r >> 3) << 2) | (r & 3);
  return (((t * 2 + s) * 2 + hf) << 3) | j;
}

// Swizzled byte offset of 16-byte block `blk` of row `row`.
template <int ROW_BYTES>
__device__ __forceinline__ int k_off(int row, int blk) {
  constexpr int mask = (ROW_BYTES / 16 < 16 ? ROW_BYTES / 16 : 16) - 1;
  return row * ROW_BYTES + ((blk ^ (row & mask)) << 4);
}
__device__ __forceinline__ int vt_off(int row, int byte_in_row) {
  const int blk = byte_in_row >> 4;
  return row * (kPfKeys * 2) + (((blk ^ ((row + (row >> 3)) & 7)) << 4) | (byte_in_row & 15));
}

}  // namespace

bool prefill_supported(int kv_dtype, int q_dtype, int head_dim, int nq_rows, int block_size) {
  return (kv_dtype == kBF16 || kv_dtype == kF16) && q_dtype == kv_dtype &&
         (head_dim == 64 || head_dim == 128) && nq_rows >= kPrefillMinRows && block_size % kPfKeys == 0;
}

int prefill_nsplit(const AttendParams& p) {
  const int64_t units = (int64_t)p.num_segments * p.num_kv_heads * prefill_qtiles(p);
  const int64_t max_tiles = (int64_t)p.total_blocks * (p.block_size / kPfKeys);
  int64_t ns = (2 * 256 + units - 1) / units;  // about two workgroups per CU
  ns = ns < 1 ? 1 : (ns > kPrefillMaxSplit ? kPrefillMaxSplit : ns);
  const int64_t by_tiles = max_tiles / 8 > 0 ? max_tiles / 8 : 1;  // at least ~8 tiles per split
  return (int)(ns < by_tiles ? ns : by_tiles);
}

int64_t prefill_partial_floats(const AttendParams& p) {
  return (int64_t)p.nsplit * p.num_segments * p.num_kv_heads * prefill_rows_pad(p) * p.head_dim;
}

template <int DT, int D>
__global__ __launch_bounds__(kPfMaxThreads, 2) void attend_prefill_kernel(AttendParams p) {
  using M = Mma<DT>;
  constexpr int kPfThreads = prefill_waves(D) * kWave;
  constexpr int kPfRows = prefill_tile_rows(D);
  constexpr int DS = D / 16;                 // d slices of Q K^T
  constexpr int DTN = D / 32;                // 32-row d tiles of O^T
  constexpr int KROW = D * 2;                // bytes per K row in LDS
  constexpr int KCH = kPfKeys * D / 8 / kPfThreads;  // 16-byte K chunks per thread
  constexpr int KPT = kPfKeys * (D / 8) / kPfThreads;  // keys per thread in the V transpose (2)
  constexpr int NDCH = D / 8;                // 16-byte chunks per row
  static_assert(KCH >= 1 && (KPT == 2 || KPT == 4), "unsupported head_dim");

  constexpr int KBYTES = kPfKeys * KROW;     // one K tile in LDS
  constexpr int VBYTES = D * kPfKeys * 2;    // one V^T tile in LDS
  // Two buffers each (separate objects, so the compiler sees that loads into
  // one never alias reads of the other): while tile j's softmax and P V run,
  // tile j+1's K is already in LDS for its Q K^T, and K_{j+2} and V_{j+1} go
  // to the buffers tile j-1 has released -- one barrier per tile.
  __shared__ __align__(16) char s_k0[KBYTES];
  __shared__ __align__(16) char s_k1[KBYTES];
  __shared__ __align__(16) char s_v0[VBYTES];
  __shared__ __align__(16) char s_v1[VBYTES];

  const int nq_rows = prefill_rows(p);
  const int nqt = (nq_rows + kPfRows - 1) / kPfRows;
  // XCD-aware order: workgroups are dispatched round-robin over the 8 XCDs,
  // so the query tiles of one (segment, kv head, split) -- which read the same
  // K/V tiles -- are given consecutive slots on one XCD and share its L2.
  int id = blockIdx.x;
  if ((gridDim.x & 7) == 0) id = (id & 7) * (int)(gridDim.x >> 3) + (id >> 3);
  const int qt = id % nqt; id /= nqt;
  const int split = id % p.nsplit; id /= p.nsplit;
  const int h = id % p.num_kv_heads;
  const int seg = id / p.num_kv_heads;
  const int list = seg * p.num_kv_heads + h;

  const int off = p.cu_blocks ? p.cu_blocks[seg] : 0;
  const int nbs = p.cu_blocks ? p.cu_blocks[seg + 1] - off : p.total_blocks;
  // Counts and list entries are clamped into the segment, so a malformed list
  // never addresses outside the caches.
  const int count = min(max(p.per_head ? p.counts[list] : p.counts[seg], 0), nbs);
  const int tpb = p.block_size / kPfKeys;
  const int ntiles = count * tpb;
  const int per = (ntiles + p.nsplit - 1) / p.nsplit;
  const int t0 = min(split * per, ntiles);
  const int n = min(t0 + per, ntiles) - t0;  // tiles of this split
  const bool uni = (p.uniform != nullptr) && (p.uniform[list] != 0);
  const int* idx = p.indices + (p.per_head ? (int64_t)h * p.total_blocks : 0) + off;

  const int t = threadIdx.x;
  const int lane = t & (kWave - 1);
  const int wave = t / kWave;
  const int hf = lane >> 5;
  const int q32 = lane & 31;

  // Q^T slices (B operand): row r, 8 dims at 16 ds + 8 hf.  A uniform list
  // takes equal logits: zero query fragments make every S entry exactly 0.
  const int row = qt * kPfRows + wave * 32 + q32;
  u32x4_t qf[DS];
  {
    const int rc = min(row, nq_rows - 1);
    const int st = rc / p.group, g = rc - st * p.group;
    const char* qp = reinterpret_cast<const char*>(p.q) +
                     ((int64_t)seg * p.q_seg_stride + (int64_t)st * p.q_tok_stride +
                      (int64_t)(h * p.group + g) * p.q_head_stride + 8 * hf) * 2;
#pragma unroll
    for (int ds = 0; ds < DS; ++ds) {
      qf[ds] = ld16v(qp + ds * 32);
      if (uni) qf[ds] = u32x4_t{0u, 0u, 0u, 0u};
    }
  }

  const int64_t krow_g = p.k_tok_stride * 2, vrow_g = p.v_tok_stride * 2;
  const char* kbase = reinterpret_cast<const char*>(p.k) + (int64_t)h * p.k_head_stride * 2;
  const char* vbase = reinterpret_cast<const char*>(p.v) + (int64_t)h * p.v_head_stride * 2;

  // This thread's share of a tile: K chunks c = t + kPfThreads u, loaded straight
  // into LDS (lane l of a wave writes 16 bytes at the instruction's base +
  // 16 l), so LDS chunk c -- row c / NDCH, swizzled position c % NDCH -- is
  // fetched from the global chunk the swizzle puts there; V keys
  // vk0 .. vk0 + KPT - 1 at chunk vdch, through registers for the transpose.
  // Lane -> (16-byte chunk, key group) of the V transpose (two keys per
  // thread, one 4-byte write per dim).  For head_dim 128 the 32 lanes of an
  // LDS write phase cover 8 dims (8 rows of V^T, whose swizzles differ) x the
  // 4 key pairs of one 16-byte block position, i.e. 32 distinct banks; a
  // wave still reads whole 256-byte key rows.  (The previous map put only 8
  // banks under a phase: 16% bank-conflict cycles, no measurable time.)
  int vdch, vgrp;
  if constexpr (NDCH == 16) {
    static_assert(kPfThreads == 512 && KPT == 2, "lane map for 512 threads, two keys each");
    vdch = (t & 7) | (((t >> 5) & 1) << 3);
    vgrp = ((t >> 3) & 1) | (((t >> 6) & 1) << 1) | (((t >> 4) & 1) << 2) | (((t >> 7) & 3) << 3);
  } else {
    vdch = t % NDCH;
    vgrp = t / NDCH;
  }
  const int vk0 = vgrp * KPT;
  // Byte offsets inside a tile (64 token rows), fixed per thread.
  int koff[KCH], voff[KPT];
#pragma unroll
  for (int u = 0; u < KCH; ++u) {
    const int c = t + kPfThreads * u;
    constexpr int mask = (NDCH < 16 ? NDCH : 16) - 1;
    const int r = c / NDCH;
    koff[u] = (int)(r * krow_g) + (((c % NDCH) ^ (r & mask)) << 4);
  }
#pragma unroll
  for (int i = 0; i < KPT; ++i) voff[i] = (int)((vk0 + i) * vrow_g) + vdch * 16;
  // First token of the split's tile j.  List and page entries are read with
  // scalar loads (the tile is the same for the whole workgroup), which do not
  // wait behind the tile loads in flight.
  auto tile_tok = [&](int j) -> int64_t {
    const int tau = t0 + j;
    const int blk = min(max(ld_const(idx + tau / tpb), 0), nbs - 1);
    int64_t page = (int64_t)off + blk;
    if (p.pages) {
      const int pg = ld_const(p.pages + page);
      page = (unsigned)pg < (unsigned)p.num_pages ? pg : (pg < 0 ? 0 : p.num_pages - 1);
    }
    return page * p.block_size + (int64_t)(tau % tpb) * kPfKeys;
  };
  u32x4_t vr[KPT];
  const int wbase = __builtin_amdgcn_readfirstlane(wave) * kWave * 16;
  auto load_k = [&](int64_t tok, char* sk) {
    const char* kt = kbase + tok * krow_g;
#pragma unroll
    for (int u = 0; u < KCH; ++u)
      __builtin_amdgcn_global_load_lds((const void*)(kt + koff[u]),
                                       (__attribute__((address_space(3))) void*)(sk + u * kPfThreads * 16 + wbase),
                                       16, 0, 0);
  };
  auto load_v = [&](int64_t tok) {
    const char* vt = vbase + tok * vrow_g;
#pragma unroll
    for (int i = 0; i < KPT; ++i) vr[i] = ld16v(vt + voff[i]);
  };
  // V^T: element e of the chunk is dim 8 vdch + e; the KPT keys are adjacent
  // in vt_pos order, so each dim takes one 4- or 8-byte write.
  auto store_v = [&](char* sv) {
    const int pb = vt_pos(vk0) * 2;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const int w = e >> 1;
      const bool hi = e & 1;
      uint32_t pk[KPT / 2];
#pragma unroll
      for (int i = 0; i < KPT / 2; ++i) {
        const uint32_t a = vr[2 * i][w], b = vr[2 * i + 1][w];
        pk[i] = hi ? ((a >> 16) | (b & 0xffff0000u)) : ((a & 0xffffu) | (b << 16));
      }
      char* dst = sv + vt_off(8 * vdch + e, pb);
      if constexpr (KPT == 4) {
        *reinterpret_cast<uint2*>(dst) = make_uint2(pk[0], pk[1]);
      } else {
        *reinterpret_cast<uint32_t*>(dst) = pk[0];
      }
    }
  };
  // S^T for the two 32-key halves of a tile, the two MFMA chains interleaved
  // over the d slices.
  auto qk = [&](const char* sk, f32x16_t (&s)[2]) {
    f32x16_t acc0, acc1;
#pragma unroll
    for (int i = 0; i < 16; ++i) { acc0[i] = 0.f; acc1[i] = 0.f; }
#pragma unroll
    for (int ds = 0; ds < DS; ++ds) {
      const u32x4_t a0 = *reinterpret_cast<const u32x4_t*>(sk + k_off<KROW>(q32, 2 * ds + hf));
      const u32x4_t a1 = *reinterpret_cast<const u32x4_t*>(sk + k_off<KROW>(32 + q32, 2 * ds + hf));
      acc0 = M::run(a0, qf[ds], acc0);
      acc1 = M::run(a1, qf[ds], acc1);
    }
    s[0] = acc0;
    s[1] = acc1;
  };

  f32x16_t o[DTN];
#pragma unroll
  for (int dt = 0; dt < DTN; ++dt)
#pragma unroll
    for (int i = 0; i < 16; ++i) o[dt][i] = 0.f;
  float m_run = -INFINITY, l_run = 0.f;
  const float c = p.logit_scale;

  // Prologue: K_0, K_1 and V_0 in LDS, V_1 in registers, S_0.  Every
  // direct-to-LDS load has completed before the barrier that publishes it.
  f32x16_t s_cur[2], s_nxt[2];
  int64_t tok2 = 0;  // first token of tile j+2 at step j
  if (n > 0) {
    const int64_t tok0 = tile_tok(0);
    load_k(tok0, s_k0);
    const int64_t tok1 = n > 1 ? tile_tok(1) : tok0;
    if (n > 1) load_k(tok1, s_k1);
    load_v(tok0);
    store_v(s_v0);
    if (n > 1) load_v(tok1);
    if (n > 2) tok2 = tile_tok(2);
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    qk(s_k0, s_cur);
  }
  // Tile j: K_j was read by the previous tile's step, V_j and K_{j+1} are in
  // LDS.  kf / vn: the buffers to fill (K_{j+2}, V_{j+1}); kn / sv: K_{j+1}
  // and V_j.  Past the end the V store writes stale registers into a buffer
  // that is never read again, and qk computes an S that is never used.
  auto step = [&](int j, char* kf, const char* kn, char* vn, const char* sv) {
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    if (j + 2 < n) load_k(tok2, kf);
    store_v(vn);
    if (j + 2 < n) load_v(tok2);
    if (j + 3 < n) tok2 = tile_tok(j + 3);

    // Online softmax of tile j for query q32 (both lane halves hold it).
    float mx = -INFINITY;
#pragma unroll
    for (int kt = 0; kt < 2; ++kt)
#pragma unroll
      for (int i = 0; i < 16; ++i) mx = fmaxf(mx, s_cur[kt][i]);
    mx = fmaxf(mx, __shfl_xor(mx, 32, kWave));
    // Lazy rescale: the reference point m_run moves only when the tile max
    // exceeds it by more than 2^kLazy (weights stay <= 2^kLazy, exact in fp32
    // and in the bf16/fp16 P operand); l and O use the same reference, so the
    // quotient o / l is unchanged.  Most tiles then skip the O rescale.
    const float m_tile = mx * c;
    const bool move = !(m_tile <= m_run + kLazy);  // also true for the first tile (m_run = -inf)
    const float m_new = move ? fmaxf(m_run, m_tile) : m_run;
    const float alpha = (m_run == -INFINITY) ? 0.f : __builtin_amdgcn_exp2f(m_run - m_new);
    if (__ballot(move)) {  // wave-uniform
#pragma unroll
      for (int dt = 0; dt < DTN; ++dt)
#pragma unroll
        for (int i = 0; i < 16; ++i) o[dt][i] *= alpha;
    }

    // S_{j+1} (independent of this tile's softmax, so its MFMAs overlap the
    // exponentials below; the rescale branch comes first so that both are in
    // one basic block).
    qk(kn, s_nxt);
    // P^T slices for the P V product, packed to the MFMA operand type as they
    // are made; the row sum adds the packed weights (what P V multiplies).
    float psum = 0.f;
    u32x4_t pb4[4];
#pragma unroll
    for (int q4 = 0; q4 < 4; ++q4) {
      float w8[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) w8[e] = __builtin_amdgcn_exp2f(fmaf(s_cur[q4 >> 1][8 * (q4 & 1) + e], c, -m_new));
      pb4[q4] = M::pack(w8);
#pragma unroll
      for (int w = 0; w < 4; ++w) psum = dot2_acc<DT>(pb4[q4][w], kOnePair<DT>, psum);
    }
    l_run = fmaf(l_run, alpha, psum);
    m_run = m_new;

    // O^T += V^T P^T over the four 16-key slices.
#pragma unroll
    for (int kt = 0; kt < 2; ++kt) {
#pragma unroll
      for (int sl = 0; sl < 2; ++sl) {
        const int pb = (((kt * 2 + sl) * 2 + hf) << 4);
        u32x4_t va[DTN];
#pragma unroll
        for (int dt = 0; dt < DTN; ++dt) va[dt] = *reinterpret_cast<const u32x4_t*>(sv + vt_off(dt * 32 + q32, pb));
        const u32x4_t b = pb4[kt * 2 + sl];
#pragma unroll
        for (int dt = 0; dt < DTN; ++dt) o[dt] = M::run(va[dt], b, o[dt]);
      }
    }
#pragma unroll
    for (int kt = 0; kt < 2; ++kt) s_cur[kt] = s_nxt[kt];
  };
  for (int j = 0; j < n; j += 2) {
    step(j, s_k0, s_k1, s_v1, s_v0);
    if (j + 1 < n) step(j + 1, s_k1, s_k0, s_v0, s_v1);
  }

  // Partial for this split: m and l per row, O^T unnormalised.
  const float l_tot = l_run + __shfl_xor(l_run, 32, kWave);
  const int64_t rows_pad = (int64_t)nqt * kPfRows;
  const int64_t slab = ((int64_t)(split * p.num_segments + seg) * p.num_kv_heads + h);
  if (hf == 0) {
    st4_nt(p.part_ml + (slab * rows_pad + row) * 2, m_run);
    st4_nt(p.part_ml + (slab * rows_pad + row) * 2 + 1, l_tot);
  }
  float* po = p.part_o + slab * D * rows_pad + row;
#pragma unroll
  for (int dt = 0; dt < DTN; ++dt)
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const int d = dt * 32 + 8 * (i >> 2) + 4 * hf + (i & 3);
      st4_nt(po + (int64_t)d * rows_pad, o[dt][i]);
    }
}

// Merge the splits: one workgroup per (segment, kv head, 64 query rows, 16
// dims).  Thread t takes row t % 64 and dims 4 (t / 64) .. +3; every split's
// (m, l) and o values are requested before any arithmetic (split indices
// clamped, weights of missing splits zero), and the result goes through LDS
// so output rows are written with d fastest.
constexpr int kCombineDims = 16;

template <int D>
__global__ __launch_bounds__(256) void prefill_combine_kernel(AttendParams p) {
  constexpr int NS = kPrefillMaxSplit;
  __shared__ float s_o[64 * (kCombineDims + 1)];
  const int nq_rows = prefill_rows(p);
  const int64_t rows_pad = prefill_rows_pad(p);
  const int nrc = (int)(rows_pad / 64);
  constexpr int ndc = D / kCombineDims;
  int id = blockIdx.x;
  const int dc = id % ndc; id /= ndc;
  const int rc = id % nrc; id /= nrc;
  const int h = id % p.num_kv_heads;
  const int seg = id / p.num_kv_heads;
  const int t = threadIdx.x;
  const int r = t & 63;
  const int d0 = dc * kCombineDims + (t >> 6) * 4;
  const int64_t row = (int64_t)rc * 64 + r;
  const int ns = p.nsplit;
  const int64_t slab_stride = (int64_t)p.num_segments * p.num_kv_heads;
  const int64_t slab0 = (int64_t)seg * p.num_kv_heads + h;

  float mv[NS], lv[NS], ov[NS][4];
#pragma unroll
  for (int s = 0; s < NS; ++s) {
    const int64_t slab = slab0 + (int64_t)min(s, ns - 1) * slab_stride;
    const float2 ml = *reinterpret_cast<const float2*>(p.part_ml + (slab * rows_pad + row) * 2);
    mv[s] = ml.x;
    lv[s] = ml.y;
#pragma unroll
    for (int j = 0; j < 4; ++j) ov[s][j] = p.part_o[(slab * D + d0 + j) * rows_pad + row];
  }
  float mm = -INFINITY;
#pragma unroll
  for (int s = 0; s < NS; ++s) mm = fmaxf(mm, s < ns ? mv[s] : -INFINITY);
  float ll = 0.f, acc[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int s = 0; s < NS; ++s) {
    const float w = (s >= ns || mv[s] == -INFINITY) ? 0.f : exp2f(mv[s] - mm);
    if (w != 0.f) {
      ll = fmaf(lv[s], w, ll);
#pragma unroll
      for (int j = 0; j < 4; ++j) acc[j] = fmaf(ov[s][j], w, acc[j]);
    }
  }
  const float inv = ll > 0.f ? 1.f / ll : 0.f;
#pragma unroll
  for (int j = 0; j < 4; ++j) s_o[r * (kCombineDims + 1) + (t >> 6) * 4 + j] = acc[j] * inv;
  __syncthreads();
  for (int e = t; e < 64 * kCombineDims; e += 256) {
    const int rr = e / kCombineDims, dd = e - rr * kCombineDims;
    const int64_t qrow = (int64_t)rc * 64 + rr;
    if (qrow < nq_rows) {
      const int st = (int)(qrow / p.group), g = (int)(qrow - (int64_t)st * p.group);
      const int64_t o = (int64_t)seg * p.out_seg_stride + (int64_t)st * p.out_tok_stride +
                        (int64_t)(h * p.group + g) * p.out_head_stride + dc * kCombineDims + dd;
      store_elt(p.out_dtype, p.out, o, s_o[rr * (kCombineDims + 1) + dd]);
    }
  }
}

template <int DT, int D>
static hipError_t launch_prefill_t(const AttendParams& p, hipStream_t s) {
  const int nqt = prefill_qtiles(p);
  const int64_t grid = (int64_t)p.num_segments * p.num_kv_heads * nqt * p.nsplit;
  if (grid > 0) {
    hipLaunchKernelGGL((attend_prefill_kernel<DT, D>), dim3((unsigned)grid), dim3(prefill_waves(D) * kWave), 0, s, p);
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
  }
  const int64_t cgrid = (int64_t)p.num_segments * p.num_kv_heads * (prefill_rows_pad(p) / 64) * (D / kCombineDims);
  if (cgrid > 0) hipLaunchKernelGGL((prefill_combine_kernel<D>), dim3((unsigned)cgrid), dim3(256), 0, s, p);
  return hipGetLastError();
}

hipError_t launch_prefill(const AttendParams& p, hipStream_t s) {
  if (p.kv_dtype == kBF16) {
    return p.head_dim == 64 ? launch_prefill_t<kBF16, 64>(p, s) : launch_prefill_t<kBF16, 128>(p, s);
  }
  return p.head_dim == 64 ? launch_prefill_t<kF16, 64>(p, s) : launch_prefill_t<kF16, 128>(p, s);
}

}  // namespace oc
