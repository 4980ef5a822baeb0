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
// query rows per wave, so each staged K / V tile serves 256 or 128 rows)
// takes one query tile of a (segment, kv head) and a contiguous range of the
// list's 64-key tiles (the tile range is split `nsplit` ways so the grid
// fills the chip); it writes a partial (m, l, O) per row, and
// prefill_combine_half_kernel (16-bit outputs, fp16 partials) or
// prefill_combine_kernel (fp32 outputs, fp32 partials) merges the splits.
//
// Per wave: 32 query rows, one per lane pair (lane l and l^32 hold row l%32).
// With v_mfma_f32_32x32x16 (A 32x16, B 16x32, fp32 C 32x32):
//   S^T = K Q^T   A = K tile rows from LDS (16 B per lane), B = Q^T slice from
//                 registers (loaded once), C lane l, i -> key 8(i/4)+4(l/32)+i%4,
//                 query l%32;
//   O^T += V^T P^T  A = V^T read from the natural V tile with the transposing
//                 LDS read ds_read_b64_tr_b16, B = P^T straight from the S^T
//                 registers (converted to bf16/fp16), C -> d, query l%32.
// So every query's softmax state (m, l) and its column of O^T stay in the two
// lanes that own the query: no shuffles except one xor-32 per tile for the row
// max.  The MFMA k index of P^T / V^T is a permutation of the 16 keys of a
// slice (the keys a lane holds in S^T); the transposing reads fetch V's keys
// in that order.
//
// LDS: three K tiles [64 keys][D] and three V tiles [64 keys][D], both
// loaded straight from global memory (global_load_lds), 16-byte blocks
// XOR-swizzled by row so the operand reads spread over the banks.  At tile
// step j the loads of K_{j+3} and V_{j+2} are issued while K_{j+1} and V_j
// are read, so every load has two steps to land.
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

// Swizzled byte offset of 16-byte block `blk` of row `row`.
template <int ROW_BYTES>
__device__ __forceinline__ int k_off(int row, int blk) {
  constexpr int mask = (ROW_BYTES / 16 < 16 ? ROW_BYTES / 16 : 16) - 1;
  return row * ROW_BYTES + ((blk ^ (row & mask)) << 4);
}

// Swizzle of the natural V tile in LDS: 16-byte block b of key row r sits at
// position b ^ vt_swizzle(r).  The transposing operand reads of one MFMA take
// 8 rows (row & 3 = 0..3, twice) x 64 bytes; with these swizzles they cover
// every bank exactly twice (rows of 256 bytes for head_dim 128; of 128 bytes,
// two to a bank row, for 64).
template <int D>
__host__ __device__ constexpr int vt_swizzle(int r) {
  return D == 128 ? 4 * (r & 3) : 4 * ((r >> 1) & 1);
}

typedef short v4i16_t __attribute__((ext_vector_type(4)));

// ds_read_b64_tr_b16: the 64-bit transposing LDS read of gfx950.
__device__ __forceinline__ v4i16_t ld_tr16(const char* lds_byte_addr) {
  return __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) v4i16_t*)(lds_byte_addr));
}

// s_waitcnt operand: vmcnt <= 4, expcnt and lgkmcnt not waited for.
constexpr unsigned kVmcntLe4 = 4u | (7u << 4) | (15u << 8);

// A global -> LDS load of 16 bytes per lane (global_load_lds_dwordx4: lane l
// writes 16 bytes at LDS address m0 + 16 l), written as inline assembly so
// that the compiler does not track its LDS write.  It cannot tell the six
// tile buffers apart and would otherwise wait for every load in flight
// (vmcnt(0)) before each step's LDS reads; the kernel orders these loads
// itself (s_waitcnt vmcnt, a barrier per step, vmcnt(0) before it ends).
// One wait state separates the M0 write from the load.
__device__ __forceinline__ void g2lds16(const void* gaddr, const void* lds) {
  const uint32_t m0 = __builtin_amdgcn_readfirstlane(
      (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) void*)lds);
  asm volatile("s_mov_b32 m0, %1\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, off" : : "v"(gaddr), "s"(m0) : "memory", "m0");
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
  constexpr int KROW = D * 2;                // bytes per K / V row in LDS
  constexpr int NDCH = D / 8;                // 16-byte chunks per row
  constexpr int KCH = kPfKeys * NDCH / kPfThreads;  // 16-byte chunks per thread of a K or V tile
  static_assert(KCH == 2, "two 16-byte chunks of K and two of V per thread and tile");
  constexpr int TBYTES = kPfKeys * KROW;     // one K or V tile in LDS

  // Three buffers each, as separate objects, so the compiler sees that the
  // direct-to-LDS loads into one never alias reads of another.  At tile step
  // j, K_{j+1} (for S_{j+1}) and V_j (for P_j V_j) are read while K_{j+2} and
  // V_{j+1} are in flight and K_{j+3} and V_{j+2} are requested into the
  // buffers that K_j and V_{j-1} released: every load has two steps to land.
  __shared__ __align__(16) char s_k0[TBYTES];
  __shared__ __align__(16) char s_k1[TBYTES];
  __shared__ __align__(16) char s_k2[TBYTES];
  __shared__ __align__(16) char s_v0[TBYTES];
  __shared__ __align__(16) char s_v1[TBYTES];
  __shared__ __align__(16) char s_v2[TBYTES];

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

  // This thread's share of a tile: chunks c = t + kPfThreads u, loaded straight
  // into LDS (lane l of a wave writes 16 bytes at the instruction's base +
  // 16 l), so LDS chunk c -- row c / NDCH, swizzled position c % NDCH -- is
  // fetched from the global chunk the swizzle puts there.  K blocks are
  // XOR-swizzled by row & 15 (conflict-free 16-byte operand reads); V blocks
  // by vt_swizzle (conflict-free transposing operand reads, below).
  int koff[KCH], voff[KCH];
#pragma unroll
  for (int u = 0; u < KCH; ++u) {
    const int c = t + kPfThreads * u;
    constexpr int mask = (NDCH < 16 ? NDCH : 16) - 1;
    const int r = c / NDCH;
    koff[u] = (int)(r * krow_g) + (((c % NDCH) ^ (r & mask)) << 4);
    voff[u] = (int)(r * vrow_g) + (((c % NDCH) ^ vt_swizzle<D>(r)) << 4);
  }
  // First token of the split's tile j (clamped to the last tile: the loads
  // past the end re-read it into buffers that are never consumed).  List and
  // page entries are read with scalar loads (the tile is the same for the
  // whole workgroup), which do not wait behind the tile loads in flight.
  auto tile_tok = [&](int j) -> int64_t {
    const int tau = t0 + min(j, n - 1);
    const int blk = min(max(ld_const(idx + tau / tpb), 0), nbs - 1);
    int64_t page = (int64_t)off + blk;
    if (p.pages) {
      const int pg = ld_const(p.pages + page);
      page = (unsigned)pg < (unsigned)p.num_pages ? pg : (pg < 0 ? 0 : p.num_pages - 1);
    }
    return page * p.block_size + (int64_t)(tau % tpb) * kPfKeys;
  };
  const int wbase = __builtin_amdgcn_readfirstlane(wave) * kWave * 16;
  auto load_k = [&](int64_t tok, char* sk) {
    const char* kt = kbase + tok * krow_g;
#pragma unroll
    for (int u = 0; u < KCH; ++u) g2lds16(kt + koff[u], sk + u * kPfThreads * 16 + wbase);
  };
  auto load_v = [&](int64_t tok, char* sv) {
    const char* vt = vbase + tok * vrow_g;
#pragma unroll
    for (int u = 0; u < KCH; ++u) g2lds16(vt + voff[u], sv + u * kPfThreads * 16 + wbase);
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
  // V^T operands by transposing reads of the natural V tile.  The P V
  // product takes, at slice s (keys 16 s .. 16 s + 15), lane l's 8 keys
  // 16 s + 8 (j / 4) + 4 hf + j % 4 (j = 0..7: the keys lane l holds in S^T)
  // of dim 32 dt + l % 32.  ds_read_b64_tr_b16 gives lane i of a 16-lane
  // group element i % 4 of the rows addressed by lanes i / 4 + 4 e (e = 0..3)
  // (pinned by an in-bounds probe on the box), so when group lane 4 m + a
  // addresses row kb + m, dims base + 4 a .. + 3, lane i receives keys kb ..
  // kb + 3 of dim base + i: two reads (kb = 16 s + 4 hf and 16 s + 8 + 4 hf)
  // form the operand.  Rows 16 s + 8 rr + 4 hf + m all have row & 3 = m, so
  // the lane's swizzled offset is fixed per d tile.
  int vt_lane[DTN];
  {
    const int m4 = (lane & 15) >> 2, a = lane & 3, g1 = (lane >> 4) & 1;
    const int lane_base = (4 * hf + m4) * KROW + 32 * g1 + 8 * a;
    const int sw = vt_swizzle<D>(m4) >> 2;  // the swizzle of rows with row & 3 = m4, in units of 4 blocks
#pragma unroll
    for (int dt = 0; dt < DTN; ++dt) vt_lane[dt] = lane_base + 64 * (dt ^ sw);
  }

  f32x16_t o[DTN];
#pragma unroll
  for (int dt = 0; dt < DTN; ++dt)
#pragma unroll
    for (int i = 0; i < 16; ++i) o[dt][i] = 0.f;
  float m_run = -INFINITY, l_run = 0.f;
  const float c = p.logit_scale;

  // Prologue: K_0, K_1, K_2 and V_0, V_1 requested, all landed before S_0.
  f32x16_t s_cur[2], s_nxt[2];
  int64_t tok_k = 0, tok_v = 0;  // tiles to request at the next step: K_{j+3}, V_{j+2}
  if (n > 0) {
    const int64_t tok0 = tile_tok(0), tok1 = tile_tok(1), tok2 = tile_tok(2);
    load_k(tok0, s_k0);
    load_k(tok1, s_k1);
    load_k(tok2, s_k2);
    load_v(tok0, s_v0);
    load_v(tok1, s_v1);
    tok_v = tok2;
    tok_k = tile_tok(3);
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    qk(s_k0, s_cur);
  }
  // Tile step j: kc holds K_{j+1}, vc V_j; kf and vf (K_j's and V_{j-1}'s
  // buffers) receive K_{j+3} and V_{j+2}.  Each step requests exactly four
  // 16-byte loads per thread, so waiting until at most four are outstanding
  // lands everything requested before the previous step.
  auto step = [&](int j, char* kf, const char* kc, char* vf, const char* vc) {
    if (j > 0) __builtin_amdgcn_s_waitcnt(kVmcntLe4);
    lds_barrier();
    load_k(tok_k, kf);
    load_v(tok_v, vf);
    tok_v = tok_k;
    tok_k = tile_tok(j + 4);

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
    qk(kc, s_nxt);
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
    for (int s4 = 0; s4 < 4; ++s4) {
      u32x4_t va[DTN];
#pragma unroll
      for (int dt = 0; dt < DTN; ++dt) {
        const v4i16_t r0 = ld_tr16(vc + 16 * s4 * KROW + vt_lane[dt]);
        const v4i16_t r1 = ld_tr16(vc + (16 * s4 + 8) * KROW + vt_lane[dt]);
        const uint2 w0 = __builtin_bit_cast(uint2, r0), w1 = __builtin_bit_cast(uint2, r1);
        va[dt] = u32x4_t{w0.x, w0.y, w1.x, w1.y};
      }
      const u32x4_t b = pb4[s4];
#pragma unroll
      for (int dt = 0; dt < DTN; ++dt) o[dt] = M::run(va[dt], b, o[dt]);
    }
#pragma unroll
    for (int kt = 0; kt < 2; ++kt) s_cur[kt] = s_nxt[kt];
  };
  for (int j = 0; j < n; j += 3) {
    step(j, s_k0, s_k1, s_v2, s_v0);
    if (j + 1 < n) step(j + 1, s_k1, s_k2, s_v0, s_v1);
    if (j + 2 < n) step(j + 2, s_k2, s_k0, s_v1, s_v2);
  }
  // The last steps' loads (re-reads of the last tile) land before the
  // workgroup can release its LDS.
  __builtin_amdgcn_s_waitcnt(0);

  // Partial for this split: m and l per row, O^T unnormalised.  fp32
  // outputs take fp32 O^T ([D][rows] per slab, so each store of a wave
  // writes two 128-byte row runs) and (m, l) in part_ml.  16-bit outputs take
  // O / s in fp16, row-major ([rows][D] per slab), s = the row's largest |o|
  // (1 when that is 0 or infinite), and one 16-byte record (m, l, s, 0) per
  // row after the last slab: half the bytes for the combine to read, in
  // whole 16-byte pieces of a row, and an error of at most 2^-12 s per value
  // before the weights (under the 2^-9 of a bf16 output and of the bf16 P
  // that P V multiplies).
  const float l_tot = l_run + __shfl_xor(l_run, 32, kWave);
  const int64_t rows_pad = (int64_t)nqt * kPfRows;
  const int64_t slab = ((int64_t)(split * p.num_segments + seg) * p.num_kv_heads + h);
  if (p.out_dtype == kF32) {
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
  } else {
    float mx = 0.f;
#pragma unroll
    for (int dt = 0; dt < DTN; ++dt)
#pragma unroll
      for (int i = 0; i < 16; ++i) mx = fmaxf(mx, fabsf(o[dt][i]));
    mx = fmaxf(mx, __shfl_xor(mx, 32, kWave));
    const float sc = (mx > 0.f && mx < INFINITY) ? mx : 1.f;
    const float inv = 1.f / sc;
    const int64_t nslab = (int64_t)p.nsplit * p.num_segments * p.num_kv_heads;
    if (hf == 0) {
      const float4 rec = make_float4(m_run, l_tot, sc, 0.f);
      st16_nt(p.part_o + nslab * (D / 2) * rows_pad + (slab * rows_pad + row) * 4, rec);
    }
    // Stage the wave's 32 rows in LDS (the tiles' buffers are free once every
    // wave is past its last step), then write whole rows with 16-byte stores.
    // Chunk c (16 bytes) of row r sits at chunk c ^ (r % CPR) of its LDS row.
    typedef unsigned int u32x2v __attribute__((ext_vector_type(2)));
    constexpr int CPR = 2 * D / 16;
    static_assert(2 * 32 * 2 * D == TBYTES && kPfThreads / kWave <= 8, "two waves' rows per tile buffer, four buffers");
    __syncthreads();
    const int bsel = wave >> 1;
    char* sb = bsel == 0 ? s_k0 : (bsel == 1 ? s_k1 : (bsel == 2 ? s_k2 : s_v0));
    char* stg = sb + (wave & 1) * 32 * (2 * D);
#pragma unroll
    for (int dt = 0; dt < DTN; ++dt)
#pragma unroll
      for (int i = 0; i < 16; i += 4) {
        const int c16 = dt * 4 + (i >> 2);
        u32x2v w;
        w.x = f32_to_f16_bits(o[dt][i] * inv) | (f32_to_f16_bits(o[dt][i + 1] * inv) << 16);
        w.y = f32_to_f16_bits(o[dt][i + 2] * inv) | (f32_to_f16_bits(o[dt][i + 3] * inv) << 16);
        *reinterpret_cast<u32x2v*>(stg + q32 * (2 * D) + ((c16 ^ (q32 & (CPR - 1))) * 16) + 8 * hf) = w;
      }
    u32x4_t* pw = reinterpret_cast<u32x4_t*>(p.part_o) + (slab * rows_pad + (row - q32)) * CPR;
#pragma unroll
    for (int k = 0; k < 32 * CPR / kWave; ++k) {
      const int c = lane + kWave * k;
      const int r = c / CPR, e = c % CPR;
      const u32x4_t v = *reinterpret_cast<const u32x4_t*>(stg + r * (2 * D) + ((e ^ (r & (CPR - 1))) * 16));
      __builtin_nontemporal_store(v, pw + c);
    }
  }
}

// Merge the splits: one workgroup per (segment, kv head, 64 query rows, 16
// dims).  Thread t takes row t % 64 and dims 4 (t / 64) .. +3; every split's
// (m, l) and o values are requested before any arithmetic (split indices
// clamped, weights of missing splits zero), and the result goes through LDS
// so output rows are written with d fastest.  fp32 outputs (fp32 partials).
constexpr int kCombineDims = 16;
constexpr int kCombineDPT = kCombineDims / 4;  // dims per thread

template <int D>
__global__ __launch_bounds__(256) void prefill_combine_kernel(AttendParams p) {
  constexpr int NS = kPrefillMaxSplit;
  __shared__ float s_o[64 * (kCombineDims + 1)];
  const int nq_rows = prefill_rows(p);
  const int64_t rows_pad = prefill_rows_pad(p);
  const int nrc = (int)(rows_pad / 64);
  constexpr int ndc = D / kCombineDims;
  // XCD-aware order (workgroups go round-robin over the 8 XCDs): the ndc
  // workgroups of a row chunk, which read the same (m, l) values, take
  // consecutive slots on one XCD and share its L2.
  int id = blockIdx.x;
  if ((gridDim.x & 7) == 0) id = (id & 7) * (int)(gridDim.x >> 3) + (id >> 3);
  const int dc = id % ndc; id /= ndc;
  const int rc = id % nrc; id /= nrc;
  const int h = id % p.num_kv_heads;
  const int seg = id / p.num_kv_heads;
  const int t = threadIdx.x;
  const int r = t & 63;
  const int d0 = dc * kCombineDims + (t >> 6) * kCombineDPT;
  const int64_t row = (int64_t)rc * 64 + r;
  const int ns = p.nsplit;
  const int64_t slab_stride = (int64_t)p.num_segments * p.num_kv_heads;
  const int64_t slab0 = (int64_t)seg * p.num_kv_heads + h;

  float mv[NS], lv[NS], ov[NS][kCombineDPT];
#pragma unroll
  for (int s = 0; s < NS; ++s) {
    const int64_t slab = slab0 + (int64_t)min(s, ns - 1) * slab_stride;
    const float2 ml = *reinterpret_cast<const float2*>(p.part_ml + (slab * rows_pad + row) * 2);
    mv[s] = ml.x;
    lv[s] = ml.y;
#pragma unroll
    for (int j = 0; j < kCombineDPT; ++j) ov[s][j] = p.part_o[(slab * D + d0 + j) * rows_pad + row];
  }
  float mm = -INFINITY;
#pragma unroll
  for (int s = 0; s < NS; ++s) mm = fmaxf(mm, s < ns ? mv[s] : -INFINITY);
  float ll = 0.f, acc[kCombineDPT] = {};
#pragma unroll
  for (int s = 0; s < NS; ++s) {
    const float w = (s >= ns || mv[s] == -INFINITY) ? 0.f : exp2f(mv[s] - mm);
    if (w != 0.f) {
      ll = fmaf(lv[s], w, ll);
#pragma unroll
      for (int j = 0; j < kCombineDPT; ++j) acc[j] = fmaf(ov[s][j], w, acc[j]);
    }
  }
  const float inv = ll > 0.f ? 1.f / ll : 0.f;
#pragma unroll
  for (int j = 0; j < kCombineDPT; ++j) s_o[r * (kCombineDims + 1) + (t >> 6) * kCombineDPT + j] = acc[j] * inv;
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

// Merge the splits for 16-bit outputs, from the row-major fp16 partials and
// (m, l, s) records: thread = (row, 8 dims), D / 8 lanes per row, so every
// split's 16-byte load of a row piece and the row's record (one address per
// row) are coalesced, and the 8 outputs go out in one 16-byte store (scalar
// stores when the output row is not 16-byte aligned).
template <int D>
__global__ __launch_bounds__(256) void prefill_combine_half_kernel(AttendParams p) {
  constexpr int NS = kPrefillMaxSplit;
  constexpr int LPRW = D / 8;            // lanes per row
  constexpr int RPW = 256 / LPRW;        // rows per workgroup
  const int nq_rows = prefill_rows(p);
  const int64_t rows_pad = prefill_rows_pad(p);
  const int nrc = (int)(rows_pad / RPW);
  int id = blockIdx.x;
  const int rc = id % nrc; id /= nrc;
  const int h = id % p.num_kv_heads;
  const int seg = id / p.num_kv_heads;
  const int t = threadIdx.x;
  const int e = t % LPRW;
  const int64_t row = (int64_t)rc * RPW + t / LPRW;
  const int ns = p.nsplit;
  const int64_t slab_stride = (int64_t)p.num_segments * p.num_kv_heads;
  const int64_t slab0 = (int64_t)seg * p.num_kv_heads + h;
  const int64_t nslab = slab_stride * ns;
  const float4* recs = reinterpret_cast<const float4*>(p.part_o + nslab * (D / 2) * rows_pad);
  const u32x4_t* data = reinterpret_cast<const u32x4_t*>(p.part_o);
  float mv[NS], lv[NS], sv[NS];
  u32x4_t ov[NS];
#pragma unroll
  for (int s = 0; s < NS; ++s) {
    const int64_t slab = slab0 + (int64_t)min(s, ns - 1) * slab_stride;
    const float4 rec = recs[slab * rows_pad + row];
    mv[s] = rec.x; lv[s] = rec.y; sv[s] = rec.z;
    ov[s] = data[(slab * rows_pad + row) * (D / 8) + e];
  }
  float mm = -INFINITY;
#pragma unroll
  for (int s = 0; s < NS; ++s) mm = fmaxf(mm, s < ns ? mv[s] : -INFINITY);
  float ll = 0.f, acc[8] = {};
#pragma unroll
  for (int s = 0; s < NS; ++s) {
    const float w = (s >= ns || mv[s] == -INFINITY) ? 0.f : exp2f(mv[s] - mm);
    if (w != 0.f) {
      ll = fmaf(lv[s], w, ll);
      const float ws = w * sv[s];
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        acc[2 * j] = fmaf(f16_bits_to_f32(ov[s][j]), ws, acc[2 * j]);
        acc[2 * j + 1] = fmaf(f16_bits_to_f32(ov[s][j] >> 16), ws, acc[2 * j + 1]);
      }
    }
  }
  if (row < nq_rows) {
    const float inv = ll > 0.f ? 1.f / ll : 0.f;
    const int st = (int)(row / p.group), g = (int)(row - (int64_t)st * p.group);
    const int64_t o = (int64_t)seg * p.out_seg_stride + (int64_t)st * p.out_tok_stride +
                      (int64_t)(h * p.group + g) * p.out_head_stride + 8 * e;
    char* op = reinterpret_cast<char*>(p.out) + o * 2;
    if ((reinterpret_cast<uintptr_t>(op) & 15) == 0) {
      u32x4_t w;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const float a = acc[2 * j] * inv, b = acc[2 * j + 1] * inv;
        w[j] = p.out_dtype == kBF16 ? (f32_to_bf16_bits(a) | (f32_to_bf16_bits(b) << 16))
                                    : (f32_to_f16_bits(a) | (f32_to_f16_bits(b) << 16));
      }
      *reinterpret_cast<u32x4_t*>(op) = w;
    } else {
#pragma unroll
      for (int j = 0; j < 8; ++j) store_elt(p.out_dtype, p.out, o + j, acc[j] * inv);
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
  if (cgrid > 0) {
    if (p.out_dtype == kF32) {
      hipLaunchKernelGGL((prefill_combine_kernel<D>), dim3((unsigned)cgrid), dim3(256), 0, s, p);
    } else {
      const int64_t hgrid = (int64_t)p.num_segments * p.num_kv_heads * (prefill_rows_pad(p) / (256 / (D / 8)));
      hipLaunchKernelGGL((prefill_combine_half_kernel<D>), dim3((unsigned)hgrid), dim3(256), 0, s, p);
    }
  }
  return hipGetLastError();
}

hipError_t launch_prefill(const AttendParams& p, hipStream_t s) {
  if (p.kv_dtype == kBF16) {
    return p.head_dim == 64 ? launch_prefill_t<kBF16, 64>(p, s) : launch_prefill_t<kBF16, 128>(p, s);
  }
  return p.head_dim == 64 ? launch_prefill_t<kF16, 64>(p, s) : launch_prefill_t<kF16, 128>(p, s);
}

}  // namespace oc
