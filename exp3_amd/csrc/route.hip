// Routing: V1 block scores, threshold / protected selection and index lists.
//
// V1 score (upstream/flashprefill_native_forward.py:89-175 + normalize_scores
// :410-417). One workgroup per (query tile t, q head h): four waves each hold 32
// query rows of Q in registers as the MFMA A operand; the bf16 block means Kbar_j
// (B operand, 256 B per block at D = 128) arrive in chunks of 32 blocks, each
// copied once per workgroup into a ring of LDS slots by direct global->LDS loads
// and read by all four waves:
//     S[row][j] = q_row . Kbar_j          (v_mfma_f32_32x32x16_bf16, fp32 acc)
//     x = S * fp32(scale * log2 e)
// Row i of tile t is valid for block j iff i >= 128 (j + 1) - 1 and i < S. Each
// lane reduces its 16 rows of one block column to (max, sum 2^(x - max)); the
// eight partials of a chunk (4 waves x 2 lane halves) are merged in a fixed order
// after the next chunk's barrier, giving M_tj and m_tj. The normalisation
// w_j = m_tj 2^(M_tj - max_j M_tj) / (sum_j w + 1e-9) and the selection then run
// on the row held by one wave, so the raw scores never reach HBM: for the routed
// lists, a second kernel with one workgroup per (b, t) takes every head's row
// (M, m) from the tile's index slab, where the first kernel left them, and writes
// the slab's lists and mask in whole cache lines.
//
// Selection (upstream :357-407 and kernels.py:129-160) is one shared device
// routine over a score row held in LDS: threshold fp32(max * alpha), protected
// regions, causality, then an ascending compaction by wave ballots and prefix
// counts, which yields the reference's sorted index order without a sort.
#include "common.h"

namespace spx {

constexpr int kRouteThreads = 256;
constexpr int kMaxBlocks = 1024;  // 131072 tokens

enum SelectMode { kSelectV1 = 0, kSelectProtected = 1 };

struct SelectParams {
  int mode;
  int query_blocks, key_blocks;
  int sink, window, last;
  float alpha;
  int min_budget;
};

struct SelectOut {
  int64_t* indices;   // contiguous [B, QB, KB, H]
  int32_t* counts;    // contiguous [B, QB, H]
  uint8_t* mask;      // contiguous [B, QB, KB, H] (nullable)
  int64_t row_base;   // element offset of (b, t, 0, h) in indices / mask
  int64_t count_off;  // element offset of (b, t, h) in counts
  int heads;          // stride between key blocks
};

__device__ __forceinline__ float block_reduce_max(float v, float* scratch) {
  v = wave_max(v);
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  block_sync();
  if (lane == 0) scratch[wave] = v;
  block_sync();
  float r = scratch[0];
  for (int w = 1; w < (int)(blockDim.x >> 6); ++w) r = max_nan(r, scratch[w]);
  return r;
}

__device__ __forceinline__ float block_reduce_sum(float v, float* scratch) {
  v = wave_sum(v);
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  block_sync();
  if (lane == 0) scratch[wave] = v;
  block_sync();
  float r = scratch[0];
  for (int w = 1; w < (int)(blockDim.x >> 6); ++w) r += scratch[w];
  return r;
}

// Selection of one (b, t, h) score row held in LDS `row[0 .. key_blocks)`.
// Every thread of the workgroup must call it.
__device__ void select_row(const float* row, int t, const SelectParams& p, const SelectOut& o,
                           float* scratch, int* wave_counts) {
  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = tid >> 6;
  const int nwaves = blockDim.x >> 6;
  const int kb = p.key_blocks;

  float local = -INFINITY;
  for (int j = tid; j < kb; j += blockDim.x) local = max_nan(local, row[j]);
  const float maximum = block_reduce_max(local, scratch);
  const float threshold = maximum * p.alpha;   // fp32(max * fp32(alpha))
  const bool all_causal = p.mode == kSelectProtected && p.alpha == 0.0f;
  const bool last_rows = t >= p.query_blocks - p.last;

  int base = 0;
  for (int j0 = 0; j0 < kb; j0 += blockDim.x) {
    const int j = j0 + tid;
    bool active = false;
    if (j < kb) {
      const float s = row[j];
      bool keep;
      if (all_causal) {
        keep = true;
      } else if (p.mode == kSelectV1) {
        keep = s >= threshold;
        if (p.min_budget > 0) {
          // rank among the row (NaN largest, ties toward the lower key id)
          int rank = 0;
          const bool s_nan = s != s;
          for (int i = 0; i < kb; ++i) {
            const float u = row[i];
            const bool u_nan = u != u;
            bool before;
            if (u_nan || s_nan) before = u_nan && (!s_nan || i < j);
            else before = u > s || (u == s && i < j);
            rank += before ? 1 : 0;
          }
          keep = keep || rank < p.min_budget;
        }
      } else {
        keep = (s > 0.0f) && (s >= threshold);
      }
      const int distance = t - j;
      const bool prot = all_causal || j < p.sink || (distance >= 0 && distance < p.window) || last_rows;
      active = (keep || prot) && distance >= 0;
      if (o.mask) o.mask[o.row_base + (int64_t)j * o.heads] = active ? 1 : 0;
    }
    const uint64_t ballot = __ballot(active);
    const int before = __popcll(ballot & ((1ull << lane) - 1ull));
    block_sync();
    if (lane == 0) wave_counts[wave] = __popcll(ballot);
    block_sync();
    int offset = base;
    for (int w = 0; w < wave; ++w) offset += wave_counts[w];
    if (active && o.indices) o.indices[o.row_base + (int64_t)(offset + before) * o.heads] = j;
    for (int w = 0; w < nwaves; ++w) base += wave_counts[w];
  }
  if (o.indices) {
    for (int pos = base + tid; pos < kb; pos += blockDim.x)
      o.indices[o.row_base + (int64_t)pos * o.heads] = kb;
  }
  if (o.counts && tid == 0) o.counts[o.count_off] = base;
}

// Reductions over a wave with DPP row operations (quad permutes, half-row and row
// mirrors, row broadcasts 15 and 31) instead of LDS-routed lane shuffles; the
// result is read from lane 63 and is wave-uniform. Lanes a DPP step cannot source
// take `identity`.
template <class Op>
__device__ __forceinline__ float wave_reduce_dpp(float v, float identity, Op op) {
  const int id = __float_as_int(identity);
#define SPX_DPP_STEP(ctrl, rows) \
  v = op(v, __int_as_float(__builtin_amdgcn_update_dpp(id, __float_as_int(v), ctrl, rows, 0xf, false)))
  SPX_DPP_STEP(0xB1, 0xf);   // quad_perm [1, 0, 3, 2]
  SPX_DPP_STEP(0x4E, 0xf);   // quad_perm [2, 3, 0, 1]
  SPX_DPP_STEP(0x141, 0xf);  // row_half_mirror
  SPX_DPP_STEP(0x140, 0xf);  // row_mirror: every lane of a 16-lane row holds the row's value
  SPX_DPP_STEP(0x142, 0xa);  // row_bcast 15 into rows 1 and 3
  SPX_DPP_STEP(0x143, 0xc);  // row_bcast 31 into rows 2 and 3: lane 63 holds the total
#undef SPX_DPP_STEP
  return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 63));
}
__device__ __forceinline__ float wave_max_dpp(float v) {
  return wave_reduce_dpp(v, -INFINITY, [](float a, float b) { return max_nan(a, b); });
}
__device__ __forceinline__ float wave_sum_dpp(float v) {
  return wave_reduce_dpp(v, 0.0f, [](float a, float b) { return a + b; });
}

// Selection of one score row held in registers by one wave (block c * 64 + lane in
// sv[c]): the same rule as select_row, chosen by p.mode (kSelectV1: upstream
// :357-407 with min_budget = 0; kSelectProtected: kernels.py:129-151, s > 0 && s >= thr and
// every causal block at alpha 0), one ballot per 64 key blocks. Bit lane of words[c]
// says whether block c * 64 + lane is selected (c < ceil(kb / 64)); returns the count.
constexpr int kRowChunks = kMaxBlocks / 64;
template <int NC>
__device__ __forceinline__ int select_row_bits(const float (&sv)[NC], int t,
                                                  const SelectParams& p, uint64_t* words) {
  const int lane = threadIdx.x & 63;
  const int kb = p.key_blocks;
  const int nch = (kb + 63) >> 6;
  // per-lane conditions are selects, not branches (the chunk test is uniform)
  float local = -INFINITY;
#pragma unroll
  for (int c = 0; c < NC; ++c)
    if (c < nch) local = max_nan(local, c * 64 + lane < kb ? sv[c] : -INFINITY);
  const float maximum = wave_max_dpp(local);
  const float threshold = maximum * p.alpha;   // fp32(max * fp32(alpha))
  const bool last_rows = t >= p.query_blocks - p.last;
  const bool protected_mode = p.mode == kSelectProtected;
  const bool all_causal = protected_mode && p.alpha == 0.0f;
  int count = 0;
#pragma unroll
  for (int c = 0; c < NC; ++c) {
    if (c < nch) {   // wave-uniform
      const int j = c * 64 + lane;
      const bool keep = protected_mode ? (sv[c] > 0.0f && sv[c] >= threshold) : sv[c] >= threshold;
      const int distance = t - j;
      const bool prot = all_causal || j < p.sink || (distance >= 0 && distance < p.window) || last_rows;
      const bool active = j < kb && (keep || prot) && distance >= 0;
      const uint64_t ballot = __ballot(active);
      if (lane == 0) words[c] = ballot;
      count += __popcll(ballot);
    }
  }
  return count;
}

// normalize_scores (upstream :410-417) of one score row held by one wave over
// j <= t: block j = c * 64 + lane has running max mx[c] and mass ms[c] (mx -inf
// when no row of the tile is valid for it); on return mx[c] holds its normalised
// score w_j / (sum w + 1e-9), w_j = ms 2^(mx - max_j mx), and 0 beyond t. Chunks
// c >= nch are left as they are.
template <int NC>
__device__ __forceinline__ void normalize_row_regs(float (&mx)[NC], const float (&ms)[NC], int t,
                                                   int nch) {
  // per-lane conditions are selects, not branches (the chunk test is uniform):
  // fmaxf with -inf and sums with 0 leave the results unchanged
  const int lane = threadIdx.x & 63;
  float local = -INFINITY;
#pragma unroll
  for (int c = 0; c < NC; ++c)
    if (c < nch) local = fmaxf(local, c * 64 + lane <= t ? mx[c] : -INFINITY);
  const float gmax = wave_max_dpp(local);
  float wsum = 0.0f;
#pragma unroll
  for (int c = 0; c < NC; ++c) {
    if (c < nch) {
      const float e = ms[c] * exp2_fast(mx[c] - gmax);
      const float w = (c * 64 + lane <= t && mx[c] != -INFINITY) ? e : 0.0f;
      wsum += w;
      mx[c] = w;
    }
  }
  const float total = wave_sum_dpp(wsum) + 1e-9f;
#pragma unroll
  for (int c = 0; c < NC; ++c)
    if (c < nch) mx[c] = c * 64 + lane <= t ? mx[c] / total : 0.0f;
}

// ------------------------------------------------------------ V1 scores

struct V1Args {
  const uint16_t* q;
  int64_t qs_b, qs_s, qs_h;
  const uint16_t* kbar;
  int64_t ms_b, ms_j, ms_h;
  int batch, seq, q_heads, kv_heads, blocks;
  float scale_log2;
  float* score;  // nullable
  int64_t ss_b, ss_t, ss_j, ss_h;
  // fused selection (indices != nullptr)
  SelectParams sel;
  int64_t* indices;
  int32_t* counts;
  uint8_t* mask;
};

// (max, mass) of one chunk column: this lane's 16 rows of block j. Rows are valid
// for j when row_in_tile >= lim (lim = 128 (j - t) + 127, at most -1 below the
// diagonal) and row_in_tile < rows_left. With a positive scale c the row maximum
// is taken over the raw products, since rounding is monotone:
// max_r fp32(acc_r c) = fp32(max_r(acc_r) c); the exponent is then one fma.
template <bool kPosScale, bool kMasked>
__device__ __forceinline__ void chunk_column(const f32x16& acc, float c, int lim, int rows_left,
                                             int wave, int lane, float& mx, float& mass) {
  bool valid[16];
#pragma unroll
  for (int r = 0; r < 16; ++r) {
    const int row = wave * 32 + mfma32_row(r, lane);
    valid[r] = !kMasked || (row >= lim && row < rows_left);
  }
  mass = 0.0f;
  if constexpr (kPosScale) {
    float m = -INFINITY;
#pragma unroll
    for (int r = 0; r < 16; ++r) m = fmaxf(m, valid[r] ? acc[r] : -INFINITY);
    mx = m * c;
    if (mx != -INFINITY) {
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const float e = exp2_fast(fmaf(acc[r], c, -mx));
        mass += valid[r] ? e : 0.0f;
      }
    }
  } else {
    float xs[16];
    float m = -INFINITY;
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      xs[r] = valid[r] ? acc[r] * c : -INFINITY;
      m = fmaxf(m, xs[r]);
    }
    mx = m;
    if (mx != -INFINITY) {
#pragma unroll
      for (int r = 0; r < 16; ++r) mass += exp2_fast(xs[r] - mx);
    }
  }
}

// Dynamic LDS of the V1 kernel when it normalises its own row: blk_max, blk_mass [NB].
__host__ __device__ constexpr size_t v1_lds_bytes(int blocks) { return 2u * (size_t)blocks * 4u; }

// Block-mean chunks (32 blocks x D dims bf16) stream through a ring of S LDS
// slots, each copied once per workgroup by direct global->LDS loads and read by all
// four waves as MFMA B operands; S - 1 chunks are in flight ahead of the one being
// reduced.
template <int D, int S> struct V1Ring {
  static constexpr int kSlots = S;
  static constexpr int kUnitsPerRow = D / 8;                  // 16-byte units of one block row
  static constexpr int kSlotElems = 32 * D;
  static constexpr int kCopiesPerWave = 32 * kUnitsPerRow / 64 / 4;   // D/64 loads per wave
  static constexpr int kInFlight = kCopiesPerWave * (kSlots - 2);      // loads left after a chunk's wait
  static_assert(kInFlight == 2 || kInFlight == 4, "ring waits below cover 2 or 4 loads");
};

// One 16-byte unit per lane from base + byte_off (base wave-uniform, a 32-bit
// per-lane offset), landing at lds_byte + 16 * lane (lds_byte wave-uniform).
// Issued from assembly: the compiler's builtin for this load makes it treat all of
// LDS as pending and wait for every copy before the next LDS read.
__device__ __forceinline__ void v1_copy_unit(const uint16_t* base, uint32_t byte_off,
                                             uint32_t lds_byte) {
  const uint32_t m0 = __builtin_amdgcn_readfirstlane(lds_byte);
  uint32_t saved;
  asm volatile(
      "s_mov_b32 %0, m0\n\t"
      "s_mov_b32 m0, %1\n\t"
      "s_nop 0\n\t"
      "global_load_lds_dwordx4 %2, %3\n\t"
      "s_mov_b32 m0, %0"
      : "=&s"(saved)
      : "s"(m0), "v"(byte_off), "s"(base)
      : "memory");
}
// 16 bytes from this lane's own address to lds_byte + 16 * lane (lds_byte
// wave-uniform), from assembly like v1_copy_unit.
__device__ __forceinline__ void v1_gather_unit(const void* src, uint32_t lds_byte) {
  const uint32_t m0 = __builtin_amdgcn_readfirstlane(lds_byte);
  uint32_t saved;
  asm volatile(
      "s_mov_b32 %0, m0\n\t"
      "s_mov_b32 m0, %1\n\t"
      "s_nop 0\n\t"
      "global_load_lds_dwordx4 %2, off\n\t"
      "s_mov_b32 m0, %0"
      : "=&s"(saved)
      : "s"(m0), "v"(src)
      : "memory");
}
template <int N> __device__ __forceinline__ void v1_wait_ring() {
  if constexpr (N == 4) asm volatile("s_waitcnt vmcnt(4)" ::: "memory");
  else asm volatile("s_waitcnt vmcnt(2)" ::: "memory");
}
__device__ __forceinline__ void v1_wait_all() { asm volatile("s_waitcnt vmcnt(0)" ::: "memory"); }

// kSplit: the routed form. The workgroup leaves each block's (max, mass) for its
// row in the index slab of its (b, t), the [NB, Hq] int64 entries the tile's
// lists will occupy: float2 entry h * NB + j of the slab for block j <= t (row h
// contiguous), and ends; v1_select_kernel then normalises and selects every row
// of the tile and overwrites the slab with the lists, so this kernel's LDS is
// not held through that epilogue. Otherwise (scores only) wave 0 normalises the
// row from LDS and writes the scores.
template <int D, int kSlots, bool kPosScale, bool kSplit>
__global__ __launch_bounds__(kRouteThreads) void v1_route_kernel(V1Args a) {
  using Ring = V1Ring<D, kSlots>;
  constexpr int kSteps = D / 16;  // 16-dim MFMA k-steps
  constexpr int R = Ring::kSlots;
  // Workgroups go to the 8 XCDs round-robin by id: the k-th one on XCD x takes
  // (batch, head) k % per_tile of tile rank x + 8 (k / per_tile), rank 0 being
  // the heaviest (last) tile. All heads of a tile then run on one XCD, so the
  // partial cache lines of its head-interleaved index and mask rows meet in
  // one L2, and the tiles are still dealt heaviest first over the XCDs.
  const int per_tile = a.batch * a.q_heads;
  const int xcd = blockIdx.x & 7, k = blockIdx.x >> 3;
  const int rank = xcd + 8 * (k / per_tile);
  if (rank >= a.blocks) return;  // padding of the grid to 8 tile ranks
  const int t = a.blocks - 1 - rank;
  const int bh = k % per_tile;
  const int b = bh / a.q_heads, h = bh % a.q_heads;
  const int g = h / (a.q_heads / a.kv_heads);
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int col = lane & 31, half = lane >> 5;

  __shared__ __align__(16) uint16_t ring[R][Ring::kSlotElems];
  __shared__ float part_max[2][8][32];   // per lane half (max, mass) of the last two chunks
  __shared__ float part_mass[2][8][32];
  extern __shared__ float v1_lds[];
  const int nb = a.blocks;
  float* blk_max = v1_lds;
  float* blk_mass = v1_lds + nb;
  // kSplit: this row's partials in the slab of (b, t)
  const int64_t part_base = (((int64_t)b * a.blocks + t) * a.blocks) * a.q_heads + (int64_t)h * a.blocks;

  // Slot image: 16-byte unit u of block row r at unit u ^ (r & 15), so that the
  // operand reads below (32 rows, one unit each) are free of bank conflicts. Lane
  // L of a wave's i-th copy fills unit P = (4 i + wave) 64 + L of the slot; block
  // rows past the last block read the last block (masked out in the reduction).
  const uint16_t* kb_bg = a.kbar + b * a.ms_b + g * a.ms_h;
  const int block_stride = (int)a.ms_j;   // elements between blocks (checked to fit on the host)
  const uint32_t ring_lds = (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) uint16_t*)&ring[0][0];
  auto issue_chunk = [&](int jc) {
    const uint32_t slot_lds = ring_lds + (uint32_t)((jc % R) * Ring::kSlotElems * 2);
#pragma unroll
    for (int i = 0; i < Ring::kCopiesPerWave; ++i) {
      const int p0 = (i * 4 + wave) * 64;
      const int unit = p0 + lane;
      const int r = unit / Ring::kUnitsPerRow;
      const int lu = (unit % Ring::kUnitsPerRow) ^ (r & 15);
      const int j = min(jc * 32 + r, nb - 1);
      v1_copy_unit(kb_bg, (uint32_t)(j * block_stride + lu * 8) * 2u, slot_lds + (uint32_t)p0 * 16u);
    }
  };
  const int nchunks = (t + 1 + 31) / 32;
  // Q rows as A operands: lane holds row (wave * 32 + col), dims dc*16 + 8*half + 0..7.
  const int row_in_tile = wave * 32 + col;
  const int64_t qrow = (int64_t)t * kBlock + row_in_tile;
  const bool q_ok = qrow < a.seq;
  bf16x8 qa[kSteps];
  if constexpr (D == 128 && R == 4) {
    // The 32 KB Q tile fills the still empty ring exactly: copied as whole 256-byte
    // rows (16 lanes per row, unit c of row r at c ^ (r & 15)), then read into the
    // operand registers, before the first block-mean chunks are copied. Loaded
    // directly in the operand layout, each load instruction took 16 bytes of 32
    // rows: 80 -> 72 us per 32K layer with the tile through LDS.
    const uint16_t* q_bh = a.q + b * a.qs_b + h * a.qs_h;
#pragma unroll
    for (int i = 0; i < kBlock * 16 / kRouteThreads; ++i) {
      const int p = i * kRouteThreads + tid;
      const int r = p >> 4, u = (p & 15) ^ (r & 15);
      const int64_t row = min(t * kBlock + r, a.seq - 1);
      v1_gather_unit(q_bh + row * a.qs_s + u * 8,
                     ring_lds + (uint32_t)(i * kRouteThreads + wave * 64) * 16u);
    }
    v1_wait_all();
    block_sync();
    const uint16_t* qt = &ring[0][0];
#pragma unroll
    for (int dc = 0; dc < kSteps; ++dc) {
      u32x4 raw = *reinterpret_cast<const u32x4*>(
          qt + row_in_tile * D + (((2 * dc + half) ^ (row_in_tile & 15)) << 3));
      if (!q_ok) raw = u32x4{0u, 0u, 0u, 0u};
      qa[dc] = as_bf16x8(raw);
    }
    block_sync();  // every wave has its rows: the ring takes the block-mean chunks
    for (int p = 0; p < R - 1 && p < nchunks; ++p) issue_chunk(p);
  } else {
    // d = 256: the ring (3 x 16 KB) is smaller than the 64 KB tile; the first chunks
    // are copied while the rows load straight into the operand registers
    for (int p = 0; p < R - 1 && p < nchunks; ++p) issue_chunk(p);
    const uint16_t* src = a.q + b * a.qs_b + qrow * a.qs_s + h * a.qs_h + half * 8;
#pragma unroll
    for (int dc = 0; dc < kSteps; ++dc) {
      u32x4 raw = {0u, 0u, 0u, 0u};
      if (q_ok) raw = *reinterpret_cast<const u32x4*>(src + dc * 16);
      qa[dc] = as_bf16x8(raw);
    }
  }

  const float c = a.scale_log2;
  const int rows_left = a.seq - t * kBlock;               // valid rows of tile t (<= 128)
  const bool tile_full = rows_left >= kBlock;
  // this lane's operand unit for k-step dc is (2 dc + half) ^ (col & 15) = 2 dc ^ hc
  const int hc = half ^ (col & 15);
  auto process = [&](int jc) {
    const uint16_t* slot = &ring[jc % R][col * D];
    // operand reads issued a group of k-steps ahead of the dependent product chain;
    // groups of at most 8 (32 registers) keep d = 256 at three waves per SIMD
    constexpr int kGroup = kSteps < 8 ? kSteps : 8;
    f32x16 acc = {};
#pragma unroll
    for (int g0 = 0; g0 < kSteps; g0 += kGroup) {
      bf16x8 kbv[kGroup];
#pragma unroll
      for (int i = 0; i < kGroup; ++i)
        kbv[i] = *reinterpret_cast<const bf16x8*>(slot + ((2 * (g0 + i)) ^ hc) * 8);
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int i = 0; i < kGroup; ++i) acc = mfma32(qa[g0 + i], kbv[i], acc);
    }
    // acc[r] = S[row 8*(r/4) + 4*half + r%4 of this wave][block j]
    const int j = jc * 32 + col;  // this lane's block column
    float mx, mass;
    if (tile_full && jc * 32 + 31 < t) {
      chunk_column<kPosScale, false>(acc, c, 0, kBlock, wave, lane, mx, mass);
    } else {
      chunk_column<kPosScale, true>(acc, c, kBlock * (j - t) + kBlock - 1, rows_left, wave,
                                    lane, mx, mass);
    }
    // every lane half's partial (16 rows) goes to LDS; merge_chunk combines them
    part_max[jc & 1][2 * wave + half][col] = mx;
    part_mass[jc & 1][2 * wave + half][col] = mass;
  };
  // the eight partials (4 waves x 2 lane halves) of chunk jc -> the block's (max,
  // mass), in a fixed order (threads 0..31): into blk_max / blk_mass, or (kSplit)
  // into the row's index slots for j <= t
  auto merge_chunk = [&](int jc) {
    const int jj = jc * 32 + tid;
    if (tid < 32 && (kSplit ? jj <= t : jj < nb)) {
      float m = part_max[jc & 1][0][tid];
#pragma unroll
      for (int w = 1; w < 8; ++w) m = fmaxf(m, part_max[jc & 1][w][tid]);
      float s2 = 0.0f;
      if (m != -INFINITY) {   // a partial with no valid row has max -inf: 2^-inf = 0, mass 0
#pragma unroll
        for (int w = 0; w < 8; ++w)
          s2 += part_mass[jc & 1][w][tid] * exp2_fast(part_max[jc & 1][w][tid] - m);
      }
      if constexpr (kSplit) {
        reinterpret_cast<float2*>(a.indices)[part_base + jj] = make_float2(m, s2);
      } else {
        blk_max[jj] = m;
        blk_mass[jj] = s2;
      }
    }
  };
  // Q is consumed here, so the compiler's wait for it (which also covers the
  // first copies) sits before the loop rather than inside it.
#pragma unroll
  for (int dc = 0; dc < kSteps; ++dc) asm volatile("" ::"v"(qa[dc]));

  // One barrier per chunk: after it, chunk jc is in LDS for every wave, every wave
  // is done reading the slot the next copy overwrites, and the partials of chunk
  // jc - 1 are complete.
  for (int jc = 0; jc < nchunks; ++jc) {
    if (jc + R - 2 < nchunks) v1_wait_ring<Ring::kInFlight>();   // chunks jc + 1 .. jc + R - 2 stay in flight
    else v1_wait_all();
    block_sync();
    if (jc > 0) merge_chunk(jc - 1);
    if (jc + R - 1 < nchunks) issue_chunk(jc + R - 1);
    process(jc);
  }
  block_sync();
  if (nchunks > 0) merge_chunk(nchunks - 1);
  if constexpr (kSplit) return;
  block_sync();
  // Scores only: one wave normalises the row (at most NB <= 1024 entries, 16 per
  // lane, held in registers: no barriers or cross-wave reductions); the other
  // waves end here.
  if (wave != 0) return;
  const int nch = (a.blocks + 63) >> 6;
  float sv[kRowChunks], sm[kRowChunks];
#pragma unroll
  for (int c = 0; c < kRowChunks; ++c) {
    sv[c] = -INFINITY;
    sm[c] = 0.0f;
    const int jj = c * 64 + lane;
    if (c < nch && jj <= t) {
      sv[c] = blk_max[jj];
      sm[c] = blk_mass[jj];
    }
  }
  normalize_row_regs(sv, sm, t, nch);
#pragma unroll
  for (int c = 0; c < kRowChunks; ++c) {
    const int jj = c * 64 + lane;
    if (c < nch && jj < a.blocks) a.score[b * a.ss_b + t * a.ss_t + jj * a.ss_j + h * a.ss_h] = sv[c];
  }
}

// Normalisation and selection of the routed rows (upstream :410-417 and
// :357-407) from the per-block (max, mass) that v1_route_kernel<..., kSplit> left
// in the index slab of each (b, t): one workgroup per (b, t), heaviest tiles
// first. Each wave takes rows h = wave, wave + 16, ...: it loads the row's
// partials (contiguous), normalises the row in registers and records its
// selection as one ballot word per 64 key blocks in LDS. After the barrier every
// partial has been read, and the tile's [NB, Hq] index and mask slabs are
// written with consecutive lanes on consecutive entries (whole cache lines), in
// passes over groups of heads whose lists fit the LDS list buffer (one pass
// unless Hq * NB > 32768): the group's rows are compacted from their words into
// LDS lists, then entry (p, h) is the p-th selected block of row h, or NB past
// the row's count.
constexpr int kSelectThreads = 1024;
constexpr int kSelectMaxHeads = 256;
constexpr int kSelectListEntries = 32768;   // uint16 list entries in LDS (64 KB)

__host__ __device__ constexpr size_t v1_select_lds_bytes(int heads, int nc) {
  return (size_t)heads * ((size_t)nc * 8 + 4) + (size_t)kSelectListEntries * 2;
}

// The tile's outputs once every row's selection words and count are in LDS (and
// every input read): counts, then the [KB, H] index and mask slabs, in groups of
// heads whose lists fit the LDS list buffer (one group unless H * KB > 32768); each
// group's rows are compacted from their words into LDS lists, then entry (p, h) is
// the p-th selected block of row h, or KB past the row's count. Written with
// consecutive lanes on consecutive entries (whole cache lines), non-temporally (the
// slabs are read only by later launches). Null outputs are skipped.
template <int NC>
__device__ __forceinline__ void write_tile_slabs(const uint64_t* words, const int* count,
                                                 uint16_t* list, int H, int KB, int nch,
                                                 int64_t slab, int64_t count_base,
                                                 int64_t* indices, int32_t* counts,
                                                 uint8_t* mask) {
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  constexpr int kWaves = kSelectThreads / 64;
  if (counts && tid < H) counts[count_base + tid] = count[tid];
  const int group = min(H, kSelectListEntries / KB);   // >= 32 (KB <= 1024)
  const int span = kSelectThreads / group;              // positions per sweep
  const int p_off = tid / group, hl = tid - p_off * group;
  for (int h0 = 0; h0 < H; h0 += group) {
    const int gh = min(group, H - h0);
    if (indices) {
      // lists of the group's rows, compacted from their words
      for (int r = wave; r < gh; r += kWaves) {
        const uint64_t* w = words + (size_t)(h0 + r) * NC;
        int base = 0;
#pragma unroll
        for (int c = 0; c < NC; ++c) {
          if (c < nch) {
            const uint64_t m = w[c];
            if ((m >> lane) & 1ull)
              list[r * KB + base + __popcll(m & ((1ull << lane) - 1ull))] = (uint16_t)(c * 64 + lane);
            base += __popcll(m);
          }
        }
      }
    }
    block_sync();
    if (p_off < span && hl < gh) {
      const int h = h0 + hl;
      if (indices) {
        const int n = count[h];
        for (int p = p_off; p < KB; p += span)
          __builtin_nontemporal_store(p < n ? (int64_t)list[hl * KB + p] : (int64_t)KB,
                                      &indices[slab + (int64_t)p * H + h]);
      }
      if (mask) {
        const uint64_t* w = words + (size_t)h * NC;
        for (int j = p_off; j < KB; j += span)
          __builtin_nontemporal_store((uint8_t)((w[j >> 6] >> (j & 63)) & 1ull),
                                      &mask[slab + (int64_t)j * H + h]);
      }
    }
    block_sync();   // the list buffer is free for the next group
  }
}

template <int NC>   // NC >= ceil(NB / 64) chunks of 64 key blocks per row
__global__ __launch_bounds__(kSelectThreads) void v1_select_kernel(V1Args a) {
  extern __shared__ __align__(8) unsigned char sel_lds[];
  const int H = a.q_heads, NB = a.blocks;
  uint64_t* words = reinterpret_cast<uint64_t*>(sel_lds);          // [H][NC]
  int* count = reinterpret_cast<int*>(words + (size_t)H * NC);     // [H]
  uint16_t* list = reinterpret_cast<uint16_t*>(count + H);         // [group heads][NB]
  const int b = (int)blockIdx.x % a.batch;
  const int t = NB - 1 - (int)blockIdx.x / a.batch;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  constexpr int kWaves = kSelectThreads / 64;
  const int64_t slab = (((int64_t)b * NB + t) * NB) * H;
  const float2* part = reinterpret_cast<const float2*>(a.indices) + slab;
  const int nch = (NB + 63) >> 6;
  for (int h = wave; h < H; h += kWaves) {
    float sv[NC], sm[NC];
#pragma unroll
    for (int c = 0; c < NC; ++c) {
      sv[c] = -INFINITY;
      sm[c] = 0.0f;
      if (c < nch) {   // wave-uniform; lanes past t read entry t and drop it
        const int jj = c * 64 + lane;
        const float2 p = part[(int64_t)h * NB + min(jj, t)];
        sv[c] = jj <= t ? p.x : -INFINITY;
        sm[c] = jj <= t ? p.y : 0.0f;
      }
    }
    normalize_row_regs(sv, sm, t, nch);
    if (a.score) {
#pragma unroll
      for (int c = 0; c < NC; ++c) {
        const int jj = c * 64 + lane;
        if (c < nch && jj < NB) a.score[b * a.ss_b + t * a.ss_t + jj * a.ss_j + h * a.ss_h] = sv[c];
      }
    }
    const int n = select_row_bits(sv, t, a.sel, words + (size_t)h * NC);
    if (lane == 0) count[h] = n;
  }
  block_sync();   // every partial of the slab has been read
  write_tile_slabs<NC>(words, count, list, H, NB, nch, slab, ((int64_t)b * NB + t) * H, a.indices,
                       a.counts, a.mask);
}

// ------------------------------------------------------- score selection

struct SelectArgs {
  const float* score;
  int64_t ss_b, ss_t, ss_j, ss_h;
  int batch, heads;
  SelectParams sel;
  int64_t* indices;
  int32_t* counts;
  uint8_t* mask;
};

__global__ __launch_bounds__(kRouteThreads) void select_kernel(SelectArgs a) {
  const int h = blockIdx.x % a.heads;
  const int t = (blockIdx.x / a.heads) % a.sel.query_blocks;
  const int b = blockIdx.x / (a.heads * a.sel.query_blocks);
  __shared__ float row[kMaxBlocks];
  __shared__ float scratch[8];
  __shared__ int wave_counts[8];
  const int kb = a.sel.key_blocks;
  for (int j = threadIdx.x; j < kb; j += blockDim.x)
    row[j] = a.score[b * a.ss_b + t * a.ss_t + j * a.ss_j + h * a.ss_h];
  block_sync();
  SelectOut o;
  o.indices = a.indices;
  o.counts = a.counts;
  o.mask = a.mask;
  o.heads = a.heads;
  o.row_base = (((int64_t)b * a.sel.query_blocks + t) * kb) * a.heads + h;
  o.count_off = ((int64_t)b * a.sel.query_blocks + t) * a.heads + h;
  select_row(row, t, a.sel, o, scratch, wave_counts);
}

// Selection of every score row of a (b, t) at once, the same rule as select_kernel
// when min_budget is 0: one workgroup per (b, t), wave w taking heads w, w + 16, ...;
// each row is read into registers (its key blocks ss_j apart; the tile's heads share
// the cache lines), reduced to ballot words in LDS, and the tile's counts, index and
// mask slabs are written by write_tile_slabs.
template <int NC>   // NC >= ceil(KB / 64)
__global__ __launch_bounds__(kSelectThreads) void select_rows_kernel(SelectArgs a) {
  extern __shared__ __align__(8) unsigned char sel_lds[];
  const int H = a.heads, KB = a.sel.key_blocks, QB = a.sel.query_blocks;
  uint64_t* words = reinterpret_cast<uint64_t*>(sel_lds);          // [H][NC]
  int* count = reinterpret_cast<int*>(words + (size_t)H * NC);     // [H]
  uint16_t* list = reinterpret_cast<uint16_t*>(count + H);         // [group heads][KB]
  const int b = (int)blockIdx.x % a.batch;
  const int t = QB - 1 - (int)blockIdx.x / a.batch;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int nch = (KB + 63) >> 6;
  const float* row0 = a.score + b * a.ss_b + t * a.ss_t;
  for (int h = wave; h < H; h += kSelectThreads / 64) {
    float sv[NC];
#pragma unroll
    for (int c = 0; c < NC; ++c) {
      sv[c] = 0.0f;
      // lanes past the row read its last entry; the rule ignores entries j >= KB
      if (c < nch) sv[c] = row0[min(c * 64 + lane, KB - 1) * a.ss_j + h * a.ss_h];
    }
    const int n = select_row_bits(sv, t, a.sel, words + (size_t)h * NC);
    if (lane == 0) count[h] = n;
  }
  block_sync();
  write_tile_slabs<NC>(words, count, list, H, KB, nch, (((int64_t)b * QB + t) * KB) * H,
                       ((int64_t)b * QB + t) * H, a.indices, a.counts, a.mask);
}

// Mask -> sorted indices (kernels.py:154-160) reuses select_row in "all causal"
// form on a 0/1 row: keep = mask, no protection, no causality.
struct MaskArgs {
  uint8_t* mask;
  int batch, query_blocks, key_blocks, heads;
  int64_t* indices;
  int32_t* counts;
};

__global__ __launch_bounds__(kRouteThreads) void indices_from_mask_kernel(MaskArgs a) {
  const int h = blockIdx.x % a.heads;
  const int t = (blockIdx.x / a.heads) % a.query_blocks;
  const int b = blockIdx.x / (a.heads * a.query_blocks);
  const int kb = a.key_blocks;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int nwaves = blockDim.x >> 6;
  __shared__ int wave_counts[8];
  const int64_t row_base = (((int64_t)b * a.query_blocks + t) * kb) * a.heads + h;
  int base = 0;
  for (int j0 = 0; j0 < kb; j0 += blockDim.x) {
    const int j = j0 + tid;
    const bool active = j < kb && a.mask[row_base + (int64_t)j * a.heads] != 0;
    const uint64_t ballot = __ballot(active);
    const int before = __popcll(ballot & ((1ull << lane) - 1ull));
    block_sync();
    if (lane == 0) wave_counts[wave] = __popcll(ballot);
    block_sync();
    int offset = base;
    for (int w = 0; w < wave; ++w) offset += wave_counts[w];
    if (active) a.indices[row_base + (int64_t)(offset + before) * a.heads] = j;
    for (int w = 0; w < nwaves; ++w) base += wave_counts[w];
  }
  for (int pos = base + tid; pos < kb; pos += blockDim.x)
    a.indices[row_base + (int64_t)pos * a.heads] = kb;
  if (tid == 0) a.counts[((int64_t)b * a.query_blocks + t) * a.heads + h] = base;
}

// Indices -> mask (kernels.py:163-176): clear the row, then mark listed ids.
__global__ __launch_bounds__(kRouteThreads) void mask_from_indices_kernel(MaskArgs a,
                                                                          const int64_t* idx,
                                                                          const int32_t* cnt) {
  const int h = blockIdx.x % a.heads;
  const int t = (blockIdx.x / a.heads) % a.query_blocks;
  const int b = blockIdx.x / (a.heads * a.query_blocks);
  const int kb = a.key_blocks;
  const int64_t row_base = (((int64_t)b * a.query_blocks + t) * kb) * a.heads + h;
  uint8_t* mask = a.mask;
  for (int j = threadIdx.x; j < kb; j += blockDim.x) mask[row_base + (int64_t)j * a.heads] = 0;
  block_sync();
  const int count = min(max(cnt[((int64_t)b * a.query_blocks + t) * a.heads + h], 0), kb);
  for (int p = threadIdx.x; p < count; p += blockDim.x) {
    const int64_t j = idx[row_base + (int64_t)p * a.heads];
    if (j >= 0 && j < kb) mask[row_base + j * a.heads] = 1;
  }
}

}  // namespace spx

using namespace spx;

static int check_q(const char* name, const void* p, const int64_t* st) {
  SPX_REQUIRE(p != nullptr && st != nullptr, SPX_EINVAL, "%s: null pointer", name);
  SPX_REQUIRE(st[3] == 1, SPX_EINVAL, "%s: innermost (dim) stride must be 1", name);
  SPX_REQUIRE((reinterpret_cast<uintptr_t>(p) & 15) == 0, SPX_EINVAL,
              "%s: base pointer must be 16-byte aligned", name);
  SPX_REQUIRE(st[0] % 8 == 0 && st[1] % 8 == 0 && st[2] % 8 == 0, SPX_EINVAL,
              "%s: batch / sequence / head strides must be multiples of 8 elements", name);
  return SPX_OK;
}

static int v1_common(const void* q, const int64_t* q_strides, const void* mean_k,
                     const int64_t* mk_strides, int batch, int seq, int q_heads, int kv_heads,
                     int head_dim, int block_size, float scale, V1Args* a) {
  SPX_REQUIRE(head_dim == 128 || head_dim == 256, SPX_EUNSUPPORTED,
              "head_dim %d unsupported (128 or 256)", head_dim);
  SPX_REQUIRE(block_size == kBlock, SPX_EUNSUPPORTED, "block_size %d unsupported (only 128)", block_size);
  SPX_REQUIRE(batch > 0 && seq > 0 && q_heads > 0 && kv_heads > 0 && q_heads % kv_heads == 0,
              SPX_EINVAL, "bad shape: batch %d seq %d q_heads %d kv_heads %d", batch, seq,
              q_heads, kv_heads);
  const int blocks = num_blocks(seq);
  SPX_REQUIRE(blocks <= kMaxBlocks, SPX_EUNSUPPORTED, "seq %d exceeds %d blocks", seq, kMaxBlocks);
  int e = check_q("q", q, q_strides);
  if (e) return e;
  e = check_q("mean_k", mean_k, mk_strides);
  if (e) return e;
  // the block-mean copies address a block by a 32-bit byte offset from its (b, g) base
  SPX_REQUIRE(mk_strides[1] > 0 && (int64_t)blocks * mk_strides[1] * 2 < (1ll << 31), SPX_EINVAL,
              "mean_k: block stride %lld must be positive and keep %d blocks within 2 GiB",
              (long long)mk_strides[1], blocks);
  a->q = static_cast<const uint16_t*>(q);
  a->qs_b = q_strides[0]; a->qs_s = q_strides[1]; a->qs_h = q_strides[2];
  a->kbar = static_cast<const uint16_t*>(mean_k);
  a->ms_b = mk_strides[0]; a->ms_j = mk_strides[1]; a->ms_h = mk_strides[2];
  a->batch = batch; a->seq = seq; a->q_heads = q_heads; a->kv_heads = kv_heads;
  a->blocks = blocks;
  a->scale_log2 = (float)((double)scale * 1.4426950408889634);
  return SPX_OK;
}

// One workgroup per (query tile, batch, q head), the tile count padded to a
// multiple of 8 (the XCD count). Scores only: LDS sized to the block count (at
// most 40 KB at 1024 blocks), the row normalised in the same launch. Routed:
// the select kernel follows on the same stream. A positive scale takes the row
// maxima over the raw products; any other scale (zero, negative, NaN) scales
// every product first.
template <int D, int kSlots, bool kSplit>
static void launch_v1_as(const V1Args& a, hipStream_t st) {
  const int tiles8 = 8 * ((a.blocks + 7) / 8);
  const int grid = tiles8 * a.batch * a.q_heads;
  const size_t lds = kSplit ? 0 : v1_lds_bytes(a.blocks);
  if (a.scale_log2 > 0.0f) v1_route_kernel<D, kSlots, true, kSplit><<<grid, kRouteThreads, lds, st>>>(a);
  else v1_route_kernel<D, kSlots, false, kSplit><<<grid, kRouteThreads, lds, st>>>(a);
  if (kSplit) {
    const int nch = (a.blocks + 63) / 64;
    const int grid = a.blocks * a.batch;
    const int h = a.q_heads;
    constexpr int T = kSelectThreads;
    if (nch <= 1) v1_select_kernel<1><<<grid, T, v1_select_lds_bytes(h, 1), st>>>(a);
    else if (nch <= 2) v1_select_kernel<2><<<grid, T, v1_select_lds_bytes(h, 2), st>>>(a);
    else if (nch <= 4) v1_select_kernel<4><<<grid, T, v1_select_lds_bytes(h, 4), st>>>(a);
    else if (nch <= 8) v1_select_kernel<8><<<grid, T, v1_select_lds_bytes(h, 8), st>>>(a);
    else v1_select_kernel<16><<<grid, T, v1_select_lds_bytes(h, 16), st>>>(a);
  }
}

static void launch_v1(const V1Args& a, int head_dim, void* stream) {
  const hipStream_t st = static_cast<hipStream_t>(stream);
  const bool split = a.indices != nullptr;
  if (head_dim == 128) {
    if (split) launch_v1_as<128, 4, true>(a, st);
    else launch_v1_as<128, 4, false>(a, st);
  } else {
    if (split) launch_v1_as<256, 3, true>(a, st);
    else launch_v1_as<256, 3, false>(a, st);
  }
}

extern "C" int spx_v1_scores(const void* q, const int64_t* q_strides, const void* mean_k,
                             const int64_t* mean_k_strides, int batch, int seq, int q_heads,
                             int kv_heads, int head_dim, int block_size, float scale,
                             float* score, const int64_t* score_strides, void* stream) {
  V1Args a{};
  int e = v1_common(q, q_strides, mean_k, mean_k_strides, batch, seq, q_heads, kv_heads,
                    head_dim, block_size, scale, &a);
  if (e) return e;
  SPX_REQUIRE(score && score_strides, SPX_EINVAL, "score: null pointer");
  a.score = score;
  a.ss_b = score_strides[0]; a.ss_t = score_strides[1]; a.ss_j = score_strides[2];
  a.ss_h = score_strides[3];
  launch_v1(a, head_dim, stream);
  return launch_status("v1_scores");
}

extern "C" int spx_v1_route(const void* q, const int64_t* q_strides, const void* mean_k,
                            const int64_t* mean_k_strides, int batch, int seq, int q_heads,
                            int kv_heads, int head_dim, int block_size, float scale, float alpha,
                            int attention_sink, int window, int last_n_blocks_full, float* score,
                            int64_t* indices, int32_t* counts, uint8_t* mask, void* stream) {
  V1Args a{};
  int e = v1_common(q, q_strides, mean_k, mean_k_strides, batch, seq, q_heads, kv_heads,
                    head_dim, block_size, scale, &a);
  if (e) return e;
  SPX_REQUIRE(indices && counts, SPX_EINVAL, "indices / counts: null pointer");
  SPX_REQUIRE(q_heads <= kSelectMaxHeads, SPX_EUNSUPPORTED, "q_heads %d exceeds %d", q_heads,
              kSelectMaxHeads);
  SPX_REQUIRE((reinterpret_cast<uintptr_t>(indices) & 7) == 0, SPX_EINVAL,
              "indices: base pointer must be 8-byte aligned");
  a.score = score;
  const int64_t nb = a.blocks;
  a.ss_h = 1; a.ss_j = q_heads; a.ss_t = nb * q_heads; a.ss_b = nb * nb * q_heads;
  a.sel.mode = kSelectV1;
  a.sel.query_blocks = a.blocks;
  a.sel.key_blocks = a.blocks;
  a.sel.sink = attention_sink;
  a.sel.window = window;
  a.sel.last = last_n_blocks_full;
  a.sel.alpha = alpha;
  a.sel.min_budget = 0;
  a.indices = indices;
  a.counts = counts;
  a.mask = mask;
  launch_v1(a, head_dim, stream);
  return launch_status("v1_route");
}

static int launch_select(int mode, const float* score, const int64_t* score_strides, int batch,
                         int query_blocks, int key_blocks, int heads, int sink, int window,
                         float alpha, int last, int min_budget, int64_t* indices,
                         int32_t* counts, uint8_t* mask, void* stream) {
  SPX_REQUIRE(score && score_strides, SPX_EINVAL, "score: null pointer");
  SPX_REQUIRE(batch > 0 && query_blocks > 0 && key_blocks > 0 && heads > 0, SPX_EINVAL,
              "bad score shape [%d, %d, %d, %d]", batch, query_blocks, key_blocks, heads);
  SPX_REQUIRE(key_blocks <= kMaxBlocks, SPX_EUNSUPPORTED, "key_blocks %d exceeds %d",
              key_blocks, kMaxBlocks);
  SPX_REQUIRE(min_budget >= 0, SPX_EINVAL, "min_budget must be >= 0");
  SelectArgs a{};
  a.score = score;
  a.ss_b = score_strides[0]; a.ss_t = score_strides[1]; a.ss_j = score_strides[2];
  a.ss_h = score_strides[3];
  a.batch = batch;
  a.heads = heads;
  a.sel.mode = mode;
  a.sel.query_blocks = query_blocks;
  a.sel.key_blocks = key_blocks;
  a.sel.sink = sink;
  a.sel.window = window;
  a.sel.last = last;
  a.sel.alpha = alpha;
  a.sel.min_budget = min_budget;
  a.indices = indices;
  a.counts = counts;
  a.mask = mask;
  const hipStream_t st = static_cast<hipStream_t>(stream);
  if (min_budget == 0 && heads <= kSelectMaxHeads) {
    const int nch = (key_blocks + 63) / 64;
    const int grid = batch * query_blocks;
    constexpr int T = kSelectThreads;
    if (nch <= 1) select_rows_kernel<1><<<grid, T, v1_select_lds_bytes(heads, 1), st>>>(a);
    else if (nch <= 2) select_rows_kernel<2><<<grid, T, v1_select_lds_bytes(heads, 2), st>>>(a);
    else if (nch <= 4) select_rows_kernel<4><<<grid, T, v1_select_lds_bytes(heads, 4), st>>>(a);
    else if (nch <= 8) select_rows_kernel<8><<<grid, T, v1_select_lds_bytes(heads, 8), st>>>(a);
    else select_rows_kernel<16><<<grid, T, v1_select_lds_bytes(heads, 16), st>>>(a);
  } else {
    // the min_budget rank (or more than 256 heads): one workgroup per row
    select_kernel<<<batch * query_blocks * heads, kRouteThreads, 0, st>>>(a);
  }
  return launch_status("select");
}

extern "C" int spx_deal_output_score(const float* score, const int64_t* score_strides, int batch,
                                     int query_blocks, int key_blocks, int heads,
                                     int attention_sink, int window, float alpha,
                                     int last_n_blocks_full, int min_budget, int64_t* indices,
                                     int32_t* counts, uint8_t* mask, void* stream) {
  SPX_REQUIRE(indices && counts, SPX_EINVAL, "indices / counts: null pointer");
  return launch_select(kSelectV1, score, score_strides, batch, query_blocks, key_blocks, heads,
                       attention_sink, window, alpha, last_n_blocks_full, min_budget, indices,
                       counts, mask, stream);
}

extern "C" int spx_protected_selection(const float* score, const int64_t* score_strides,
                                       int batch, int query_blocks, int key_blocks, int heads,
                                       float alpha, int sink_blocks, int window_blocks,
                                       int last_full_blocks, uint8_t* mask, int64_t* indices,
                                       int32_t* counts, void* stream) {
  SPX_REQUIRE(mask != nullptr, SPX_EINVAL, "mask: null pointer");
  SPX_REQUIRE((indices == nullptr) == (counts == nullptr), SPX_EINVAL,
              "indices and counts must both be given or both be null");
  return launch_select(kSelectProtected, score, score_strides, batch, query_blocks, key_blocks,
                       heads, sink_blocks, window_blocks, alpha, last_full_blocks, 0, indices,
                       counts, mask, stream);
}

extern "C" int spx_indices_from_mask(const uint8_t* mask, int batch, int query_blocks,
                                     int key_blocks, int heads, int64_t* indices,
                                     int32_t* counts, void* stream) {
  SPX_REQUIRE(mask && indices && counts, SPX_EINVAL, "null pointer");
  SPX_REQUIRE(batch > 0 && query_blocks > 0 && key_blocks > 0 && heads > 0, SPX_EINVAL,
              "bad mask shape");
  MaskArgs a{const_cast<uint8_t*>(mask), batch, query_blocks, key_blocks, heads, indices, counts};
  indices_from_mask_kernel<<<batch * query_blocks * heads, kRouteThreads, 0,
                             static_cast<hipStream_t>(stream)>>>(a);
  return launch_status("indices_from_mask");
}

extern "C" int spx_mask_from_indices(const int64_t* indices, const int32_t* counts, int batch,
                                     int query_blocks, int key_blocks, int heads, uint8_t* mask,
                                     void* stream) {
  SPX_REQUIRE(mask && indices && counts, SPX_EINVAL, "null pointer");
  SPX_REQUIRE(batch > 0 && query_blocks > 0 && key_blocks > 0 && heads > 0, SPX_EINVAL,
              "bad index shape");
  MaskArgs a{mask, batch, query_blocks, key_blocks, heads, nullptr, nullptr};
  mask_from_indices_kernel<<<batch * query_blocks * heads, kRouteThreads, 0,
                             static_cast<hipStream_t>(stream)>>>(a, indices, counts);
  return launch_status("mask_from_indices");
}
