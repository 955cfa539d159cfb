// Block-sparse causal flash attention (bf16 MFMA, fp32 online softmax in base 2)
// with an optional fused block-mean correction.
//
// Semantics follow upstream/flashprefill_native_forward.py:215-354 (_flash_forward):
// for query tile t and head h, walk the first counts[t, h] entries of the tile's
// index list in order; every listed 128-key block j contributes all its keys
// (keys past the sequence end read as zero), causality is applied only inside the
// block j == t; O = softmax(scale q K^T) V is stored as bf16 and the natural-log
// LSE = M ln 2 + ln l. List entries outside [0, NB) are skipped; a block listed
// n times is attended n times, as the reference's list walk does. With the mean
// correction, each row also attends to the fp32 block-mean key of every block
// j < t missing from its list (logit + ln n_j) with the block-mean value, inside
// the same online softmax; this equals the logaddexp merge of kernels.py:179-230
// (mean_tail) and :312-325 (merge_exact_mean).
//
// gfx950 design
//   * One workgroup (8 waves) per (pair of adjacent query tiles t, t - 1; q head):
//     waves 0-3 own the 128 rows of tile t, waves 4-7 those of tile t - 1, 32 rows
//     each. The two tiles' block lists are merged, so every K/V tile copied into
//     LDS serves both (the lists differ by little: sinks, window and most routed
//     blocks are shared); a block repeated in a list is repeated in the merged one.
//   * Scores are computed transposed, S^T = K Q^T, with v_mfma_f32_32x32x16_bf16:
//     each lane owns one query column, so row max / row sum are in-lane reductions
//     plus one exchange with the other lane half, the O rescale is a per-lane
//     scalar, and the probabilities already sit in the B-operand layout of
//     O^T = V^T P^T (no shuffles, no LDS round trip for P).
//   * K rows and the pre-transposed value tile come from the pooling pass already
//     in LDS order (XOR-swizzled 16-byte chunks, conflict-free operand reads) and
//     are copied with direct global->LDS loads into double buffers: block u + 1
//     lands while block u is computed.
//   * Full blocks are software-pipelined over their four 32-key sub-blocks (matrix
//     work of one sub-block around the exponentials of the previous one); the
//     running max moves lazily (only by more than 2^64), so the O rescale is a
//     rarely taken wave-uniform branch. The diagonal blocks (t and t - 1) run last
//     through a masked path in which wave w touches only key sub-blocks 0 .. w.
//   * Grid order: (tile pair, q head) items heaviest-first. Workgroup i runs on XCD
//     i % 8; a (batch, kv group) stream is served by a fixed set of XCDs, so the q
//     heads sharing a KV block read it from the same L2s, and with 8 / (B * Hkv)
//     XCDs per stream the heads of each tile pair are dealt over that set in turn,
//     which keeps the XCDs' shares of the work equal. Given a work queue, the grid
//     is persistent: one workgroup per CU takes its XCD's items in that order from
//     a counter, then the light last third of the tile pairs from a shared one.
#include <type_traits>

#include "common.h"

namespace spx {

constexpr int kAttnThreads = 512;     // 8 waves: two query tiles x 4 waves x 32 rows
constexpr int kItemWaves = 4;        // waves per query tile
constexpr int kMaxBlocksAttn = 1024;
constexpr int kListLoads = kMaxBlocksAttn / kAttnThreads;  // list positions per thread
constexpr int kTailTile = 64;        // mean keys per tail tile (hi and lo rows fill K LDS)
// log2 headroom before a column's running max moves. P is bf16 and O, l are fp32, all
// with an 8-bit exponent, so probabilities up to 2^64 lose nothing; O then keeps
// 2^128 / (2^64 * 2^17 keys at the 131072-token limit) = 2^47 of headroom for |v|.
// Sharp score profiles (routed sparse layers) move a column's maximum by tens of
// log2 units from block to block: at a headroom of 2^8 the rescale branch ran in
// about half of a sparse layer's sub-blocks, at 2^64 in under 3 %.
constexpr float kLazyRescale = 64.0f;

struct AttnArgs {
  const uint16_t* q;
  int64_t qs_b, qs_s, qs_h;
  const uint16_t* kt;  // key tiles   [B, Hkv, NB, 128, D]  (LDS order, from the pool pass)
  const uint16_t* vt;  // value tiles [B, Hkv, NB, D, 128]
  const int64_t* idx;  // nullable: all causal blocks
  int64_t is_b, is_t, is_p, is_h;
  const int32_t* cnt;
  int64_t cs_b, cs_t, cs_h;
  const float* mean_k;  // [B, NB, Hkv, D]
  const float* mean_v;
  const int32_t* bcounts;  // [NB]
  const uint8_t* choice;   // rescue token per (b, t, j, h): [B, NB, NB, Hq]
  const uint16_t* v;       // V [B, S, Hkv, D] (strided): rescue tokens' value rows
  int64_t vs_b, vs_s, vs_h;
  int tail_kind;           // 0 block means, 1 rescue token, 2 rescue token + remainder mean
  void* out;
  int64_t os_b, os_s, os_h;
  float* lse;  // nullable
  int64_t ls_b, ls_s, ls_h;
  int batch, seq, q_heads, kv_heads, blocks, group, num_pairs;
  int xcds_per_stream;   // XCDs sharing one (batch, kv group) stream; 1: pair p on XCD p % 8
  float scale_log2;
  // Persistent grid (a caller queue): one workgroup per CU takes items until none
  // are left. Tile pairs [0, static_tp) are dealt to XCDs as in the static grid and
  // taken in order through XCD x's counter queue[1 + x]; the rest (the lightest) go
  // through queue[0] in heaviest-first order to whichever XCD asks first.
  int* queue;        // SPX_WORK_QUEUE_INTS zeroed int32 (null: one workgroup per item)
  int static_tp;     // tile pairs on the per-XCD deal (all of them without a queue)
  int dyn_items;     // (tile pair, stream, head) items of the shared tail
};

__device__ __forceinline__ int swz(int row, int chunk) {
  return row * kBlock + ((chunk ^ (row & 15)) << 3);
}

__device__ __forceinline__ bf16x8 lds_read16(const uint16_t* lds, int off) {
  return as_bf16x8(*reinterpret_cast<const u32x4*>(lds + off));
}

__device__ __forceinline__ bf16x8 pack8(const f32x16& v, int base) {
  u32x4 w;
  w[0] = pack_bf16x2(v[base + 0], v[base + 1]);
  w[1] = pack_bf16x2(v[base + 2], v[base + 3]);
  w[2] = pack_bf16x2(v[base + 4], v[base + 5]);
  w[3] = pack_bf16x2(v[base + 6], v[base + 7]);
  return as_bf16x8(w);
}

// The running-max rescale multiplies the O accumulators in place from inline
// assembly (tied operands keep O in its registers across the rarely taken
// branch). The compiler's hazard recognizer does not look inside asm statements,
// so the wait states an MFMA that wrote O needs before VALU access to O are issued
// here, at the top of that branch: the products into O are issued before the
// branch (their results are live on both of its paths), so these wait states sit
// between the last product and the first multiply. 19 >= the 16-pass XDL write ->
// VALU read / write requirement of the gfx940 family (the 8-pass products here
// need fewer). Not tied to O: tying it changes how the loop is scheduled.
__device__ __forceinline__ void o_settle() { asm volatile("s_nop 7\n\ts_nop 7\n\ts_nop 2"); }

// Per-wave online-softmax state for its 32 query columns.
struct WaveState {
  bf16x8 qb[8];   // Q^T B operands, dim chunk dc
  f32x16 o[4];    // O^T accumulators, dim block db
  float m;        // running max (base-2, scaled), lazily moved
  float l;        // running sum over this lane half's keys
  float neg_m;    // full blocks: -m once set (0 before)
  float thr;      // full blocks: lazy-move threshold on shifted scores (-inf before m is set)
};

// Copy one 32 KB tile, already in LDS order in global memory, into LDS with
// direct global->LDS loads: lane l of a wave lands at (wave base) + 16 l, so
// thread id moves 16-byte chunks id + 512 i. No VGPRs are used for staging;
// completion is awaited with wait_tiles() before the publishing barrier.
//
// The loads are issued from inline assembly on purpose: the compiler tracks a
// builtin LDS-DMA load as a pending write to all of LDS and then waits for it
// before the next LDS read, which would serialise the copy of block u + 1 with
// the math on block u (they use different buffers). The only consumer waits
// explicitly (wait_tiles, then a barrier).
__device__ __forceinline__ void dma_part(const uint16_t* src, uint16_t* lds, int tid, int i);

__device__ __forceinline__ void dma_tile(const uint16_t* src, uint16_t* lds, int tid) {
#pragma unroll
  for (int i = 0; i < 4; ++i) dma_part(src, lds, tid, i);
}

// Part i (0..3) of dma_tile: one quarter of the tile's 16-byte chunks.
// The part offset goes into the scalar base, so every part uses the same per-lane
// offset tid * 16 (one VGPR for all copies).
__device__ __forceinline__ void dma_part(const uint16_t* src, uint16_t* lds, int tid, int i) {
  const int w = tid >> 6;
  const uint32_t lds_base =
      (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) uint16_t*)lds;
  const int chunk0 = i * kAttnThreads + w * 64;
  const uint32_t voff = (uint32_t)tid * 16u;
  const uint32_t m0 = __builtin_amdgcn_readfirstlane(lds_base + (uint32_t)chunk0 * 16u);
  src += i * kAttnThreads * 8;
  uint32_t saved;
  asm volatile(
      "s_mov_b32 %0, m0\n\t"
      "s_mov_b32 m0, %1\n\t"
      "s_nop 0\n\t"
      "global_load_lds_dwordx4 %2, %3\n\t"
      "s_mov_b32 m0, %0"
      : "=&s"(saved)
      : "s"(m0), "v"(voff), "s"(src)
      : "memory");
}

// Per-lane gather into LDS: 16 bytes from this lane's own address land at
// lds_wave + 16 x lane, lds_wave being the same for the whole wave. Issued from
// assembly like dma_part, and awaited explicitly.
__device__ __forceinline__ void dma_gather16(const void* src, uint32_t lds_wave) {
  const uint32_t m0 = __builtin_amdgcn_readfirstlane(lds_wave);
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

// threadIdx.x behind an opaque copy: values derived from it are recomputed for
// every work item of a persistent workgroup instead of being held across items.
__device__ __forceinline__ int thread_x() { return opaque((int)threadIdx.x); }

__device__ __forceinline__ void wait_tiles() { asm volatile("s_waitcnt vmcnt(0)" ::: "memory"); }

// LDS element offset of this lane's MFMA operand row (row & 15 == col & 15 for
// every operand row it reads) with 16-byte chunk 2 x + half, for x = 0: the chunk
// for any other x is base ^ (x << 4) (XOR swizzle c ^ (row & 15), c = 2 x + half).
__device__ __forceinline__ int operand_base(int row) {
  const int lane = thread_x() & 63;
  const int col = lane & 31, half = lane >> 5;
  const int cx = (col >> 1) & 7, hb = half ^ (col & 1);
  return row * kBlock + (cx << 4) + (hb << 3);
}

// Compiler fence: nothing is scheduled across it. Keeps operand reads issued a
// step ahead of the MFMAs that consume them.
__device__ __forceinline__ void fence() { __builtin_amdgcn_sched_barrier(0); }

// S^T for NMB 32-key sub-blocks at K rows row0 + 32 mb + col (for hi/lo mean
// keys, also rows + kTailTile). The NMB (x2) operand reads of a dim chunk are
// issued one chunk ahead of their MFMAs.
template <int NMB, bool HILO>
__device__ __forceinline__ void scores(const uint16_t* kb, const WaveState& ws, int row0,
                                       f32x16 (&s)[4]) {
  constexpr int P = NMB * (HILO ? 2 : 1);
  const int col = thread_x() & 31;
  const int e0 = opaque(operand_base(row0 + col));
  auto row_off = [](int part) {
    return HILO ? ((part & 1) ? kTailTile * kBlock : 0) + (part >> 1) * 32 * kBlock
                : part * 32 * kBlock;
  };
  bf16x8 ring[2][P];
#pragma unroll
  for (int mb = 0; mb < NMB; ++mb) s[mb] = f32x16{};
#pragma unroll
  for (int p = 0; p < P; ++p) ring[0][p] = lds_read16(kb, e0 + row_off(p));
  fence();
#pragma unroll
  for (int dc = 0; dc < 8; ++dc) {
    if (dc + 1 < 8) {
      const int e = e0 ^ ((dc + 1) << 4);
#pragma unroll
      for (int p = 0; p < P; ++p) ring[(dc + 1) & 1][p] = lds_read16(kb, e + row_off(p));
    }
#pragma unroll
    for (int p = 0; p < P; ++p) {
      const int mb = HILO ? (p >> 1) : p;
      s[mb] = mfma32(ring[dc & 1][p], ws.qb[dc], s[mb]);
    }
    fence();
  }
}

// Softmax of one tile: masks (DIAG) / per-key biases (BIAS, already scaled),
// lazily moved running max, probabilities packed to bf16 B operands pb[2 mb + h],
// running sum, O rescale when any lane moved its max.
template <int NMB, bool DIAG, bool BIAS>
__device__ __forceinline__ void softmax(f32x16 (&s)[4], WaveState& ws, float scale, int q_pos,
                                        const float* bias, int bias_row0, bf16x8 (&pb)[8]) {
  const int lane = thread_x() & 63;
  float mx = -INFINITY;
#pragma unroll
  for (int mb = 0; mb < NMB; ++mb) {
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      float x = s[mb][r];
      if (BIAS) x = fmaf(x, scale, bias[bias_row0 + mb * 32 + mfma32_row(r, lane)]);
      if (DIAG && mb * 32 + mfma32_row(r, lane) > q_pos) x = -INFINITY;
      s[mb][r] = x;
      mx = fmaxf(mx, x);
    }
  }
  mx = fmaxf(mx, xor32(mx));
  const float mxs = BIAS ? mx : mx * scale;
  const float m_new = (mxs > ws.m + kLazyRescale) ? mxs : ws.m;
  if (__any(m_new != ws.m)) {
    const float corr = (m_new == ws.m) ? 1.0f : exp2_fast(ws.m - m_new);
    // in place (tied operands): O keeps its registers across the rarely taken
    // branch instead of being copied into a second set on every block
    o_settle();
#pragma unroll
    for (int db = 0; db < 4; ++db) {
#pragma unroll
      for (int r = 0; r < 16; ++r) asm volatile("v_mul_f32 %0, %0, %1" : "+v"(ws.o[db][r]) : "v"(corr));
    }
    ws.l *= corr;
    ws.m = m_new;
  }
  const float neg_m = (ws.m == -INFINITY) ? 0.0f : -ws.m;
  float sum = 0.0f;
#pragma unroll
  for (int mb = 0; mb < NMB; ++mb) {
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const float p = BIAS ? exp2_fast(s[mb][r] + neg_m) : exp2_fast(fmaf(s[mb][r], scale, neg_m));
      s[mb][r] = p;
      sum += p;
    }
    pb[2 * mb] = pack8(s[mb], 0);
    pb[2 * mb + 1] = pack8(s[mb], 8);
  }
  ws.l += sum;
}

// O^T += V^T P^T over NKC 16-key chunks (value chunks 0 .. NKC-1); the four
// value-tile reads of a chunk are issued one chunk ahead.
template <int NKC>
__device__ __forceinline__ void accumulate_pv(const uint16_t* vb, WaveState& ws,
                                              const bf16x8 (&pb)[8]) {
  const int col = thread_x() & 31;
  const int e0 = opaque(operand_base(col));
  bf16x8 ring[2][4];
#pragma unroll
  for (int db = 0; db < 4; ++db) ring[0][db] = lds_read16(vb, e0 + db * 32 * kBlock);
  fence();
#pragma unroll
  for (int kc = 0; kc < NKC; ++kc) {
    if (kc + 1 < NKC) {
      const int e = e0 ^ ((kc + 1) << 4);
#pragma unroll
      for (int db = 0; db < 4; ++db) ring[(kc + 1) & 1][db] = lds_read16(vb, e + db * 32 * kBlock);
    }
#pragma unroll
    for (int db = 0; db < 4; ++db) ws.o[db] = mfma32(ring[kc & 1][db], pb[kc], ws.o[db]);
    fence();
  }
}

// One exact block: full tiles use every key sub-block with no masking; on the
// diagonal wave w only reaches sub-blocks 0 .. w (keys above its queries are
// masked, sub-blocks beyond w are skipped entirely).
template <int NMB, bool DIAG>
__device__ __forceinline__ void exact_block(const uint16_t* kb, const uint16_t* vb, WaveState& ws,
                                            float scale, int q_pos) {
  f32x16 s[4];
  bf16x8 pb[8];
  scores<NMB, false>(kb, ws, 0, s);
  softmax<NMB, DIAG, false>(s, ws, scale, q_pos, nullptr, 0, pb);
  accumulate_pv<2 * NMB>(vb, ws, pb);
}

// ---------------------------------------------------------------- full blocks
// A full (unmasked) block, software-pipelined over its four 32-key sub-blocks so
// that each group of eight MFMAs carries about half of one sub-block's softmax:
//
//   step 0: P V of the previous full block's sub-block 3 | scores S0
//   step k: P V of sub-block k-2 (k >= 2) with the shift and max of S(k-1) |
//           lazy rescale | scores S(k) (k <= 3) with the exponentials of S(k-1)
//                                                                   (k = 1..4)
//
// Sub-block 3's P V product stays pending in registers across the next block's
// barrier. The running max moves lazily per sub-block (only when a column's
// shifted max exceeds 2^64); the rescale of O comes after the P V products that
// used the old max were issued and before any that use the new one.
//
// LDS operand addresses: entry c of a table is the byte address of 16-byte chunk
// pair c of this lane's operand row in tile buffer 0; row 32 i + col of buffer B is
// the same entry plus the immediate B * 32 KB + i * 8 KB (rows congruent mod 16
// share the swizzle), so no address arithmetic is left in the block.
struct OperandTables {
  uint32_t k[8];
  uint32_t v[8];
};

__device__ __forceinline__ uint32_t lds_address(const uint16_t* p) {
  return (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) uint16_t*)p;
}

__device__ __forceinline__ bf16x8 lds_at(uint32_t byte_address) {
  const u32x4 v =
      *reinterpret_cast<const __attribute__((address_space(3))) u32x4*>((uintptr_t)byte_address);
  return as_bf16x8(v);
}

__device__ __forceinline__ OperandTables operand_tables(const uint16_t* k0, const uint16_t* v0) {
  OperandTables t;
  const int e0 = operand_base(thread_x() & 31);
  const uint32_t kb = lds_address(k0), vb = lds_address(v0);
#pragma unroll
  for (int c = 0; c < 8; ++c) {
    const uint32_t off = (uint32_t)(e0 ^ (c << 4)) * 2u;
    t.k[c] = (uint32_t)opaque((int)(kb + off));
    t.v[c] = (uint32_t)opaque((int)(vb + off));
  }
  return t;
}

constexpr uint32_t kTileBytes = kBlock * kHeadDim * 2;  // one 32 KB K or V tile
constexpr uint32_t kRowGroupBytes = 32 * kBlock * 2;    // 32 operand rows

// key operands of sub-block mb (dim chunks 0..7)
template <int BUF>
__device__ __forceinline__ void sub_keys(const OperandTables& tb, int mb, bf16x8 (&r)[8]) {
#pragma unroll
  for (int dc = 0; dc < 8; ++dc) r[dc] = lds_at(tb.k[dc] + BUF * kTileBytes + mb * kRowGroupBytes);
}

// scores of one sub-block: S^T = K_mb Q^T (8 chained MFMAs over the dim chunks)
__device__ __forceinline__ void sub_scores(const bf16x8 (&r)[8], const WaveState& ws, f32x16& acc) {
  acc = f32x16{};
#pragma unroll
  for (int dc = 0; dc < 8; ++dc) acc = mfma32(r[dc], ws.qb[dc], acc);
}

// value operands of sub-block j: value chunks 2j, 2j+1 of every dim block
template <int BUF>
__device__ __forceinline__ void sub_values(const OperandTables& tb, int j, bf16x8 (&r)[8]) {
#pragma unroll
  for (int h = 0; h < 2; ++h)
#pragma unroll
    for (int db = 0; db < 4; ++db)
      r[h * 4 + db] = lds_at(tb.v[2 * j + h] + BUF * kTileBytes + db * kRowGroupBytes);
}

__device__ __forceinline__ void sub_pv(const bf16x8 (&r)[8], const bf16x8 (&p)[2], WaveState& ws) {
#pragma unroll
  for (int h = 0; h < 2; ++h)
#pragma unroll
    for (int db = 0; db < 4; ++db) ws.o[db] = mfma32(r[h * 4 + db], p[h], ws.o[db]);
}

// Shift one sub-block's scores in place to x = s * scale + ws.neg_m (this lane's
// 16 keys of its column) and check them against the running max. The max runs
// over the shifted values: results of arithmetic, which the compiler's max takes
// without quieting them first. The running max moves lazily: only when a
// column's x exceeds ws.thr (2^64 once set); then (rarely) O and l are rescaled
// and x shifted by the same amount. Before the first move neg_m is 0 and thr
// -inf, so the first sub-block sets the max from its own scores. The common path
// checks each lane half's own max; the column max over both halves is formed
// only in the rare branch.
__device__ __forceinline__ void shift_and_check(f32x16& sv, WaveState& ws, float scale) {
#pragma unroll
  for (int r = 0; r < 16; ++r) sv[r] = fmaf(sv[r], scale, ws.neg_m);
  // each lane half checks its own 8 + 8 keys; only when some lane exceeds the
  // threshold is the column max of both halves formed
  float mx = fmaxf(fmaxf(sv[0], sv[1]), sv[2]);
#pragma unroll
  for (int r = 3; r < 15; r += 2) mx = fmaxf(fmaxf(mx, sv[r]), sv[r + 1]);
  mx = fmaxf(mx, sv[15]);
  if (__any(mx > ws.thr)) {
    const auto sw = __builtin_amdgcn_permlane32_swap(__float_as_uint(mx), __float_as_uint(mx),
                                                     false, false);
    mx = fmaxf(__uint_as_float(sw[0]), __uint_as_float(sw[1]));
    const bool move = mx > ws.thr;
    const float d = move ? mx : 0.0f;
    // nothing is accumulated before the first move (thr -inf): O and l stay 0
    const float corr = ws.thr == -INFINITY ? 0.0f : exp2_fast(-d);
    // in place (tied operands): O keeps its registers across the rarely taken branch
    o_settle();
#pragma unroll
    for (int db = 0; db < 4; ++db) {
#pragma unroll
      for (int r = 0; r < 16; ++r) asm volatile("v_mul_f32 %0, %0, %1" : "+v"(ws.o[db][r]) : "v"(corr));
    }
    ws.l *= corr;
    ws.neg_m -= d;
    if (move) ws.thr = kLazyRescale;
#pragma unroll
    for (int r = 0; r < 16; ++r) sv[r] -= d;
  }
}

// probabilities of one sub-block (shifted scores x) as bf16 B operands; the
// running sum adds the fp32 probabilities, as upstream/flashprefill_native_forward.py
// :332-338 does (sum before the cast for the P V product), pairwise so that the
// chain into l is short. (Summing the packed bf16 pairs with v_dot2_f32_bf16 instead
// took issue cycles from the matrix products beside it: four per product halved
// their rate in a microbenchmark, while plain adds there were nearly free.)
__device__ __forceinline__ void sub_exp(const f32x16& xv, WaveState& ws, bf16x8 (&p)[2]) {
  float pair_sum[8];
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    u32x4 w;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const float a = exp2_fast(xv[8 * h + 2 * i]);
      const float b = exp2_fast(xv[8 * h + 2 * i + 1]);
      w[i] = pack_bf16x2(a, b);
      pair_sum[4 * h + i] = a + b;
    }
    p[h] = as_bf16x8(w);
  }
  const float sum = ((pair_sum[0] + pair_sum[1]) + (pair_sum[2] + pair_sum[3])) +
                    ((pair_sum[4] + pair_sum[5]) + (pair_sum[6] + pair_sum[7]));
  ws.l += sum;
}

// The copy of the next block: source tiles and the other buffers.
struct NextCopy {
  const uint16_t* k;
  const uint16_t* v;
  uint16_t* kd;
  uint16_t* vd;
  bool any;
};

// One full block in buffer BUF. The previous full block's last P V product
// (value operands rv, probabilities pend) runs first, beside this block's first
// key reads; this block's own last product is left in rv / pend. A pending
// product of zero probabilities and values (the initial state) adds nothing.
template <int BUF>
__device__ __forceinline__ void full_block(const OperandTables& tb, WaveState& ws, float scale,
                                           bf16x8 (&rv)[8], bf16x8 (&pend)[2]) {
  f32x16 s[2];
  bf16x8 p[2][2];
  bf16x8 rk[8];
  // Each operand group is read one MFMA group ahead: the key reads of step k land
  // during the P V products of step k, the value reads for step k + 1 during the
  // scores of step k. The shift and max of S(k-1) run beside the P V products,
  // its exponentials beside the scores S(k).
  sub_keys<BUF>(tb, 0, rk);
  fence();
  sub_pv(rv, pend, ws);
  sub_scores(rk, ws, s[0]);
#pragma unroll
  for (int k = 1; k <= 4; ++k) {
    fence();
    if (k <= 3) sub_keys<BUF>(tb, k, rk);
    fence();
    if (k >= 2) sub_pv(rv, p[(k - 2) & 1], ws);
    shift_and_check(s[(k - 1) & 1], ws, scale);
    fence();
    sub_values<BUF>(tb, k - 1, rv);
    fence();
    if (k <= 3) sub_scores(rk, ws, s[k & 1]);
    sub_exp(s[(k - 1) & 1], ws, p[(k - 1) & 1]);
  }
  pend[0] = p[1][0];
  pend[1] = p[1][1];
}

// Tail tile entry i, 8-dim chunk c: the key as bf16 hi + lo rows (i and 64 + i,
// 16-byte chunks at the swizzled position) and the value in slot value_slot_of_key(i)
// of each of the chunk's eight dim rows.
__device__ __forceinline__ void write_tail_entry(uint16_t* kb, uint16_t* vb, int i, int c,
                                                 const float (&mk)[8], const float (&mv)[8]) {
  u32x4 hi, lo;
#pragma unroll
  for (int x = 0; x < 4; ++x) {
    const uint32_t h2 = pack_bf16x2(mk[2 * x], mk[2 * x + 1]);
    hi[x] = h2;
    lo[x] = pack_bf16x2(mk[2 * x] - bf16_lo(h2), mk[2 * x + 1] - bf16_hi(h2));
  }
  *reinterpret_cast<u32x4*>(kb + swz(i, c)) = hi;
  *reinterpret_cast<u32x4*>(kb + swz(kTailTile + i, c)) = lo;
  const int slot = value_slot_of_key(i);
#pragma unroll
  for (int x = 0; x < 8; ++x) {
    const int d = c * 8 + x;
    vb[swz(d, slot >> 3) + (slot & 7)] = to_bf16_bits(mv[x]);
  }
}

// Block-mean tail tile: entries t0 .. t0 + 63 of `ids` (unselected blocks), key =
// fp32 mean K split into bf16 hi + lo, value = bf16 mean V, logit bias ln n_j.
// One work item per (entry, 8-dim chunk).
__device__ __forceinline__ void stage_tail(const AttnArgs& a, const int16_t* ids, int ntail, int t0,
                                           int64_t desc_base, uint16_t* kb, uint16_t* vb,
                                           float* bias, int tid0, int stride) {
  for (int e = tid0; e < kTailTile * (kHeadDim / 8); e += stride) {
    const int i = e >> 4, c = e & 15;
    const int j = (t0 + i < ntail) ? (int)ids[t0 + i] : -1;
    float mk[8] = {}, mv[8] = {};
    if (j >= 0) {
      const int64_t off = (desc_base + (int64_t)j * a.kv_heads) * kHeadDim + c * 8;
      load8(a.mean_k + off, mk);
      load8(a.mean_v + off, mv);
    }
    write_tail_entry(kb, vb, i, c, mk, mv);
    if (c == 0) bias[i] = j >= 0 ? logf((float)a.bcounts[j]) * kLog2e : -INFINITY;
  }
}

// Rescue tail tile (kernels.py:233-309): entries per block epb = 1 (the block's
// rescue token: its key row, its value, logit bias 0) or 2 (also the mean of the
// other 127 tokens: (mean * 128 - token) / 127 for key and value, bias ln 127
// log2 e). Blocks t0 .. t0 + kTailTile / epb - 1 of `ids`; layout as stage_tail.
// The token's key chunk is one 16-byte read of the pool pass's key tile, its value
// chunk one 16-byte read of its row of V (history blocks j < t are full, so the
// token is inside the sequence).
__device__ __forceinline__ void stage_rescue(const AttnArgs& a, const int16_t* ids, int ntail,
                                             int t0, int epb, int b, int g, int h, int t,
                                             uint16_t* kb, uint16_t* vb, float* bias, int tid0,
                                             int stride) {
  const int64_t tile_elems = (int64_t)kBlock * kHeadDim;
  for (int e = tid0; e < kTailTile * (kHeadDim / 8); e += stride) {
    const int i = e >> 4, c = e & 15;
    const int blk = t0 + i / epb, kind = i % epb;
    const int j = blk < ntail ? (int)ids[blk] : -1;
    float mk[8] = {}, mv[8] = {};
    float bi = -INFINITY;
    if (j >= 0) {
      const int tok = a.choice[(((int64_t)b * a.blocks + t) * a.blocks + j) * a.q_heads + h];
      const int64_t tile = (((int64_t)b * a.kv_heads + g) * a.blocks + j) * tile_elems;
      const u32x4 kraw =
          *reinterpret_cast<const u32x4*>(a.kt + tile + tok * kHeadDim + ((c ^ (tok & 15)) << 3));
      const u32x4 vraw = *reinterpret_cast<const u32x4*>(
          a.v + b * a.vs_b + ((int64_t)j * kBlock + tok) * a.vs_s + g * a.vs_h + c * 8);
      float kval[8], vval[8];
#pragma unroll
      for (int x = 0; x < 4; ++x) {
        kval[2 * x] = bf16_lo(kraw[x]);
        kval[2 * x + 1] = bf16_hi(kraw[x]);
        vval[2 * x] = bf16_lo(vraw[x]);
        vval[2 * x + 1] = bf16_hi(vraw[x]);
      }
      if (kind == 0) {
#pragma unroll
        for (int x = 0; x < 8; ++x) { mk[x] = kval[x]; mv[x] = vval[x]; }
        bi = 0.0f;
      } else {
        const int64_t off = (((int64_t)b * a.blocks + j) * a.kv_heads + g) * kHeadDim + c * 8;
        float mean_k[8], mean_v[8];
        load8(a.mean_k + off, mean_k);
        load8(a.mean_v + off, mean_v);
#pragma unroll
        for (int x = 0; x < 8; ++x) {
          mk[x] = (mean_k[x] * (float)kBlock - kval[x]) / (float)(kBlock - 1);
          mv[x] = (mean_v[x] * (float)kBlock - vval[x]) / (float)(kBlock - 1);
        }
        bi = logf((float)(kBlock - 1)) * kLog2e;
      }
    }
    write_tail_entry(kb, vb, i, c, mk, mv);
    if (c == 0) bias[i] = bi;
  }
}

// Item decode, static deal: XCD x's local item l. Every XCD serves one (batch, kv
// group) stream (or a few when there are more than 8), so the q heads sharing a KV
// block read it from one L2; tile pairs heaviest first.
__device__ __forceinline__ void static_item(const AttnArgs& a, int xcd, int local, int& pair,
                                            int& hg) {
  const int bg = a.batch * a.kv_heads;
  if (a.xcds_per_stream > 1) {
    // (batch, kv group) stream s runs on the xcds_per_stream XCDs x = s (mod bg); its
    // items k = tp * group + hg (heaviest first) are dealt over them in turn, so the
    // heads of a tile pair alternate between those XCDs and every XCD's share of
    // each stream is balanced (one stream per XCD would give it every other tile
    // pair, and the always-full last tiles all to the same XCDs)
    const int s = xcd % bg;
    const int k = local * a.xcds_per_stream + xcd / bg;
    const int tpk = k / a.group;
    hg = k - tpk * a.group;
    pair = tpk * bg + s;
  } else {
    const int pair_local = local / a.group;
    hg = local - pair_local * a.group;
    pair = pair_local * 8 + xcd;
  }
}

// Work-queue counters: [0] the shared tail (one stream per XCD or fewer XCDs than
// streams), [1 + x] XCD x's share of the static deal, [kStreamCounter0 + s] the
// tail of stream s (8 / (B * Hkv) XCDs per stream, so at most 4 streams).
constexpr int kStreamCounter0 = 9;

// Item decode, shared tail: item kd of tile pairs static_tp.., (tile pair, stream,
// head) heaviest first.
__device__ __forceinline__ void tail_item(const AttnArgs& a, int kd, int& pair, int& hg) {
  const int bg = a.batch * a.kv_heads;
  const int per_tp = bg * a.group;
  const int tpk = a.static_tp + kd / per_tp;
  const int rem = kd - (tpk - a.static_tp) * per_tp;
  hg = rem % a.group;
  pair = tpk * bg + rem / a.group;
}

// Q of a tile pair staged in LDS buffer 1 (tile t in K, tile t - 1 in V; 16-byte
// chunk c of row r at r * 16 + (c ^ (r & 15))): whole 256-byte rows per 16 lanes,
// so each copy instruction reads 8 full cache lines (loaded directly in the operand
// layout, each instruction would read 32 bytes of each of 32 rows).
__device__ __forceinline__ int q_stage_chunk(int row, int c) { return row * 16 + (c ^ (row & 15)); }

__device__ __forceinline__ void copy_q(const AttnArgs& a, int b, int h, int t0, uint16_t* k1,
                                       uint16_t* v1, int tid) {
  const int w = tid >> 6;
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const int it = i >> 2;
    const int e = (i & 3) * kAttnThreads + tid;
    const int r = e >> 4, cs = e & 15;
    const int t = t0 - it;
    int64_t qrow = (int64_t)t * kBlock + r;
    if (t < 0 || qrow >= a.seq) qrow = 0;   // a row that exists; its queries are not stored
    const uint16_t* src = a.q + b * a.qs_b + qrow * a.qs_s + h * a.qs_h + ((cs ^ (r & 15)) << 3);
    dma_gather16(src, lds_address(it ? v1 : k1) + (uint32_t)(((i & 3) * kAttnThreads + w * 64) * 16));
  }
}

template <bool EXACT, bool TAIL, bool OUT_F32>
__device__ __forceinline__ void attn_item(const AttnArgs& a, int pair, int hg);

// Workgroup i runs on XCD i % 8. Without a queue every workgroup runs the one item
// the static deal gives it. With one, the grid is persistent: launching a workgroup
// costs a few microseconds, and each XCD starts its workgroups in blockIdx order, a
// batch of four at a time (one per shader engine), so with short items CUs idled
// 11 us on average between workgroups (sparse layers). XCDs also run at different
// speeds (one launch measured a 6 % spread in their summed workgroup times); the
// shared tail lets the fast ones take more of the light items.
template <bool EXACT, bool TAIL, bool OUT_F32>
__global__ __launch_bounds__(kAttnThreads, 1) void attn_kernel(AttnArgs args) {
  const int xcd = blockIdx.x & 7;
  __shared__ int next_item;
  // thread 0's draw state, kept in LDS so that no register holds it across items:
  // this XCD's share used up; streams of the tail tried
  __shared__ int share_done, steal;
  if (threadIdx.x == 0) share_done = steal = 0;
  for (int round = 0;; ++round) {
    // The arguments are read afresh for every item through an opaque pointer, so
    // nothing derived from them is held in registers across items.
#if defined(__HIP_DEVICE_COMPILE__)
    const __attribute__((address_space(4))) AttnArgs* ap =
        (const __attribute__((address_space(4))) AttnArgs*)__builtin_amdgcn_kernarg_segment_ptr();
    asm volatile("" : "+s"(ap));
    const AttnArgs a = *ap;
#else
    const AttnArgs a = args;
#endif
    int pair, hg;
    if (a.queue == nullptr) {
      if (round > 0) break;
      static_item(a, xcd, blockIdx.x >> 3, pair, hg);
    } else {
      const int bg = a.batch * a.kv_heads;
      const int n_static = a.xcds_per_stream > 1
          ? a.static_tp * a.group / a.xcds_per_stream
          : max(0, (a.static_tp * bg - xcd + 7) / 8) * a.group;
      // With 8 / bg XCDs per stream, the tail is drawn per stream: a workgroup takes
      // its own stream's light items first (their K / V tiles are in its L2), then
      // those of the other streams once its own are gone.
      const bool per_stream = a.xcds_per_stream > 1;
      const int stream_items = (a.blocks + 1) / 2 - a.static_tp;   // tile pairs ..
      const int per_stream_items = stream_items * a.group;        // .. x heads
      if (threadIdx.x == 0) {
        int k = -1;
        if (!share_done) {
          const int d = atomicAdd(a.queue + 1 + xcd, 1);
          if (d < n_static) k = d;
          else share_done = 1;
        }
        if (k < 0 && per_stream) {
          for (; steal < bg; ++steal) {
            const int st = (xcd + steal) % bg;
            const int d = atomicAdd(a.queue + kStreamCounter0 + st, 1);
            if (d < per_stream_items) {
              k = n_static + st * per_stream_items + d;
              break;
            }
          }
        } else if (k < 0) {
          const int d = atomicAdd(a.queue, 1);
          if (d < a.dyn_items) k = n_static + d;
        }
        next_item = k;   // -1: no items left
      }
      block_sync();
      const int k = next_item;
      block_sync();  // read by every wave before thread 0 takes the next one
      if (k < 0) break;
      if (k < n_static) {
        static_item(a, xcd, k, pair, hg);
      } else if (per_stream) {
        const int st = (k - n_static) / per_stream_items;
        const int d = (k - n_static) - st * per_stream_items;
        const int tpk = a.static_tp + d / a.group;
        hg = d - (tpk - a.static_tp) * a.group;
        pair = tpk * bg + st;
      } else {
        tail_item(a, k - n_static, pair, hg);
      }
    }
    attn_item<EXACT, TAIL, OUT_F32>(a, pair, hg);
  }
}

// ---- work item: query tiles (t, t - 1) of one q head
template <bool EXACT, bool TAIL, bool OUT_F32>
__device__ __forceinline__ void attn_item(const AttnArgs& a, int pair, int hg) {
  if (pair >= a.num_pairs) return;
  const int bg = a.batch * a.kv_heads;
  const int tp = pair / bg;                          // tile pair: tiles NB-1-2tp, NB-2-2tp
  const int b = (pair % bg) / a.kv_heads;
  const int g = (pair % bg) % a.kv_heads;
  const int h = g * a.group + hg;

  __shared__ __align__(16) uint16_t kbuf[2][kBlock * kBlock];
  __shared__ __align__(16) uint16_t vbuf[2][kBlock * kBlock];
  // union of both lists, ascending; a block listed n times for an item appears
  // max over the items of n times, occurrence k flagged for the items listing it
  // more than k times (the reference attends a repeated list entry repeatedly)
  __shared__ int16_t ulist[2 * kMaxBlocksAttn];
  __shared__ uint8_t uflag[2 * kMaxBlocksAttn];      // bit i: occurrence is item i's
  __shared__ uint32_t mult[2][kMaxBlocksAttn / 2];   // per-item times listed, 16 bits per block
  __shared__ float tail_bias[2][kTailTile];
  __shared__ int wave_counts[kAttnThreads / 64];

  const int tid = thread_x();
  const int lane = tid & 63;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int item = w >> 2;                           // 0: tile t, 1: tile t - 1
  const int wi = w & 3;                              // wave inside its item
  const int col = lane & 31, half = lane >> 5;
  const int q_pos = wi * 32 + col;                   // this lane's query inside its tile
  const float scale = a.scale_log2;
  const int t_item[2] = {a.blocks - 1 - 2 * tp, a.blocks - 2 - 2 * tp};
  const int t = t_item[item];                        // may be -1 (odd tile count)
  const bool live = t >= 0;

  copy_q(a, b, h, t_item[0], kbuf[1], vbuf[1], tid);   // read after the list phase
  // Both items' list counts and entries are loaded now, with the Q copy in flight. Each
  // thread reads its positions of the row clamped to the last counted one (rows and
  // positions clamped into range, so no branch separates the loads): positions past
  // the count re-read that entry's cache line instead of fetching the rest of the row
  // (heads interleave, so each position is its own line), and are dropped below.
  int count_of[2] = {0, 0};
  int64_t entry[2][kListLoads];
  if (a.idx) {
#pragma unroll
    for (int it = 0; it < 2; ++it) {
      const int tt = max(t_item[it], 0);
      count_of[it] = a.cnt[b * a.cs_b + tt * a.cs_t + h * a.cs_h];
      const int64_t* list = a.idx + b * a.is_b + tt * a.is_t + h * a.is_h;
      const int last = min(max(count_of[it], 1), a.blocks) - 1;
#pragma unroll
      for (int r = 0; r < kListLoads; ++r)
        entry[it][r] = list[min(tid + r * kAttnThreads, last) * a.is_p];
    }
  }
  WaveState ws;
  {
    ws.m = -INFINITY;
    ws.l = 0.0f;
    ws.neg_m = 0.0f;
    ws.thr = -INFINITY;
#pragma unroll
    for (int db = 0; db < 4; ++db) ws.o[db] = f32x16{};
  }

  // ---- how often each block is listed for each item (valid ids), then the union
  for (int x = tid; x < kMaxBlocksAttn; x += kAttnThreads) (&mult[0][0])[x] = 0u;
  block_sync();
#pragma unroll
  for (int it = 0; it < 2; ++it) {
    const int tt = t_item[it];
    if (tt < 0) continue;
    if (a.idx) {
      const int count = min(max(count_of[it], 0), a.blocks);   // tt >= 0 here
#pragma unroll
      for (int r = 0; r < kListLoads; ++r) {
        const int64_t j = entry[it][r];   // range-checked before narrowing
        if (tid + r * kAttnThreads < count && j >= 0 && j < a.blocks)
          atomicAdd(&mult[it][j >> 1], 1u << ((j & 1) * 16));
      }
    } else {
      for (int j = tid; j <= tt; j += kAttnThreads) atomicAdd(&mult[it][j >> 1], 1u << ((j & 1) * 16));
    }
  }
  wait_tiles();   // this wave's share of the Q copy (visible to all after the barrier)
  block_sync();
  {
    const uint16_t* qs = item ? vbuf[1] : kbuf[1];
#pragma unroll
    for (int dc = 0; dc < 8; ++dc)
      ws.qb[dc] = as_bf16x8(*reinterpret_cast<const u32x4*>(qs + q_stage_chunk(q_pos, 2 * dc + half) * 8));
  }
  // Processing order: every listed block except the two diagonal ones (t, t - 1),
  // ascending, then the diagonal ones. The block loop for the first part has a
  // single (unmasked) code path, which keeps O in one register set.
  auto times_listed = [&](int it, int j) {
    return (int)((mult[it][j >> 1] >> ((j & 1) * 16)) & 0xffffu);
  };
  int nu = 0;
  for (int j0 = 0; j0 < a.blocks; j0 += kAttnThreads) {
    const int j = j0 + tid;
    int c0 = 0, c1 = 0;
    if (j < a.blocks && j != t_item[0] && j != t_item[1]) {
      c0 = times_listed(0, j);
      c1 = times_listed(1, j);
    }
    const int e = max(c0, c1);   // occurrences of block j in the union
    int incl = e;                // inclusive prefix sum over the wave
#pragma unroll
    for (int d = 1; d < 64; d <<= 1) {
      const int v = __shfl_up(incl, d);
      if (lane >= d) incl += v;
    }
    if (lane == 63) wave_counts[w] = incl;
    block_sync();
    int offset = nu + incl - e;
    for (int x = 0; x < w; ++x) offset += wave_counts[x];
    for (int k = 0; k < e; ++k) {
      ulist[offset + k] = (int16_t)j;
      uflag[offset + k] = (uint8_t)((c0 > k ? 1 : 0) | (c1 > k ? 2 : 0));
    }
    for (int x = 0; x < kAttnThreads / 64; ++x) nu += wave_counts[x];
    block_sync();
  }
  const int n_full = __builtin_amdgcn_readfirstlane(nu);
  // the diagonal blocks t - 1, t (known ids) go after the others, ascending
  if (tid == 0) {
    int n = nu;
#pragma unroll
    for (int i = 1; i >= 0; --i) {
      const int j = t_item[i];
      if (j < 0) continue;
      const int c0 = times_listed(0, j), c1 = times_listed(1, j);
      for (int k = 0; k < max(c0, c1); ++k, ++n) {
        ulist[n] = (int16_t)j;
        uflag[n] = (uint8_t)((c0 > k ? 1 : 0) | (c1 > k ? 2 : 0));
      }
    }
    wave_counts[0] = n;
  }
  block_sync();
  nu = __builtin_amdgcn_readfirstlane(wave_counts[0]);
  if (EXACT && nu > 0) {
    const int64_t tile_elems = (int64_t)kBlock * kHeadDim;
    const uint16_t* kbase = a.kt + (((int64_t)b * a.kv_heads + g) * a.blocks) * tile_elems;
    const uint16_t* vbase = a.vt + (((int64_t)b * a.kv_heads + g) * a.blocks) * tile_elems;
    {
      const int j0 = __builtin_amdgcn_readfirstlane(ulist[0]);
      dma_tile(kbase + j0 * tile_elems, kbuf[0], tid);
      dma_tile(vbase + j0 * tile_elems, vbuf[0], tid);
    }
    // Publish block u (its copy was issued one step earlier) and start the copy of
    // block u + 1 into the other buffers, where it lands during block u's math.
    auto begin_block = [&](int u) {
      wait_tiles();
      block_sync();  // block u visible to all; every wave is done with block u - 1
      if (u + 1 < nu) {
        const int jn = __builtin_amdgcn_readfirstlane(ulist[u + 1]);
        dma_tile(kbase + jn * tile_elems, kbuf[(u + 1) & 1], tid);
        dma_tile(vbase + jn * tile_elems, vbuf[(u + 1) & 1], tid);
      }
    };
    const OperandTables tables = operand_tables(kbuf[0], vbuf[0]);
    int u = 0;
    bf16x8 rv[8], pend[2];  // the pending P V product of the last full block
#pragma unroll
    for (int i = 0; i < 8; ++i) rv[i] = bf16x8{};
    pend[0] = pend[1] = bf16x8{};
    // Full blocks: publish block u, then run it while its successor is copied (by
    // full_block, spread over its steps; here at once if this item skips block u).
    auto run_full = [&](int uu, auto buf) {
      constexpr int B = decltype(buf)::value;
      // list entries first (written before the loop): their LDS reads overlap the wait
      const int f = __builtin_amdgcn_readfirstlane(uflag[uu]);
      const bool more = uu + 1 < nu;
      const int jn = __builtin_amdgcn_readfirstlane(ulist[more ? uu + 1 : uu]);
      wait_tiles();
      block_sync();  // block uu visible to all; every wave is done with block uu - 1
      NextCopy nx;
      nx.any = more;
      nx.k = kbase + jn * tile_elems;
      nx.v = vbase + jn * tile_elems;
      nx.kd = kbuf[B ^ 1];
      nx.vd = vbuf[B ^ 1];
      if (nx.any) {  // block uu + 1 lands in the other buffers during block uu's math
        dma_tile(nx.k, nx.kd, tid);
        dma_tile(nx.v, nx.vd, tid);
      }
      if ((f >> item) & 1) full_block<B>(tables, ws, scale, rv, pend);
    };
    for (; u < n_full; u += 2) {  // unrolled by two: each block's buffer is a constant
      run_full(u, std::integral_constant<int, 0>{});
      if (u + 1 < n_full) run_full(u + 1, std::integral_constant<int, 1>{});
    }
    sub_pv(rv, pend, ws);
    if (ws.thr != -INFINITY) ws.m = -ws.neg_m;  // the max the full blocks settled on
    u = n_full;
    for (; u < nu; ++u) {
      const int cur = u & 1;
      const int j = __builtin_amdgcn_readfirstlane(ulist[u]);
      const int f = __builtin_amdgcn_readfirstlane(uflag[u]);
      begin_block(u);
      if ((f >> item) & 1) {
        if (j != t) {
          exact_block<4, false>(kbuf[cur], vbuf[cur], ws, scale, q_pos);
        } else {
          switch (wi) {  // wave wi reaches key sub-blocks 0 .. wi of the diagonal block
            case 0: exact_block<1, true>(kbuf[cur], vbuf[cur], ws, scale, q_pos); break;
            case 1: exact_block<2, true>(kbuf[cur], vbuf[cur], ws, scale, q_pos); break;
            case 2: exact_block<3, true>(kbuf[cur], vbuf[cur], ws, scale, q_pos); break;
            default: exact_block<4, true>(kbuf[cur], vbuf[cur], ws, scale, q_pos); break;
          }
        }
      }
    }
    block_sync();  // every wave is done with the last block
  }

  if (TAIL) {
    // tail of item i: {j < t_i : not listed for i}, ascending. Both items' tails
    // are staged side by side (item i uses buffer i) and processed together.
    __shared__ int16_t tlist[2][kMaxBlocksAttn];
    int ntail[2] = {0, 0};
#pragma unroll
    for (int it = 0; it < 2; ++it) {
      const int tt = t_item[it];
      for (int j0 = 0; j0 < max(tt, 0); j0 += kAttnThreads) {
        const int j = j0 + tid;
        const bool in_tail = j < tt && times_listed(it, j) == 0;
        const uint64_t ballot = __ballot(in_tail);
        const int before = __popcll(ballot & ((1ull << lane) - 1ull));
        if (lane == 0) wave_counts[w] = __popcll(ballot);
        block_sync();
        int offset = ntail[it];
        for (int x = 0; x < w; ++x) offset += wave_counts[x];
        if (in_tail) tlist[it][offset + before] = (int16_t)j;
        for (int x = 0; x < kAttnThreads / 64; ++x) ntail[it] += wave_counts[x];
        block_sync();
      }
    }
    const int64_t desc_base = (int64_t)b * a.blocks * a.kv_heads + g;  // (b, 0, g)
    const int nmax = max(ntail[0], ntail[1]);
    const int epb = a.tail_kind == 2 ? 2 : 1;   // tail entries per unselected block
    for (int t0 = 0; t0 < nmax; t0 += kTailTile / epb) {
      block_sync();
      if (a.tail_kind == 0)
        stage_tail(a, tlist[item], ntail[item], t0, desc_base, kbuf[item], vbuf[item],
                   tail_bias[item], tid & (kItemWaves * 64 - 1), kItemWaves * 64);
      else
        stage_rescue(a, tlist[item], ntail[item], t0, epb, b, g, h, t, kbuf[item], vbuf[item],
                     tail_bias[item], tid & (kItemWaves * 64 - 1), kItemWaves * 64);
      block_sync();
      if (t0 < ntail[item]) {
        f32x16 s[4];
        bf16x8 pb[8];
        scores<2, true>(kbuf[item], ws, 0, s);
        softmax<2, false, true>(s, ws, scale, q_pos, tail_bias[item], 0, pb);
        accumulate_pv<4>(vbuf[item], ws, pb);
      }
    }
  }
  // ---- epilogue (lane values re-derived: nothing is kept across the block loops)
  const float l = ws.l + xor32(ws.l);
  const bool any = l > 0.0f;
  const float inv = any ? 1.0f / l : 0.0f;
  const int tx = thread_x();
  const int half_e = (tx >> 5) & 1;
  const int wq = (tx >> 6) & 3;                       // wave inside its item
  const int64_t qrow = (int64_t)t * kBlock + wq * 32 + (tx & 31);
  if (OUT_F32) {
    if (live && qrow < a.seq) {
      float* dst = static_cast<float*>(a.out) + b * a.os_b + qrow * a.os_s + h * a.os_h;
#pragma unroll
      for (int db = 0; db < 4; ++db) {
#pragma unroll
        for (int rr = 0; rr < 4; ++rr) {
          const int d0 = db * 32 + 8 * rr + 4 * half_e;
          *reinterpret_cast<f32x4*>(dst + d0) =
              f32x4{ws.o[db][4 * rr] * inv, ws.o[db][4 * rr + 1] * inv, ws.o[db][4 * rr + 2] * inv,
                    ws.o[db][4 * rr + 3] * inv};
        }
      }
    }
  } else {
    // Each lane holds 4-dim pieces of its query row, so stored directly every store
    // instruction would write 16 bytes into each of 32 rows (cache lines). The wave
    // stages its 32 x 128 bf16 tile in LDS (8 KB per wave in the K buffers, 16-byte
    // chunk c of row r at c ^ (r & 15)) and stores whole rows: 16 lanes per 256-byte
    // row, 8 store instructions per wave.
    block_sync();   // every wave is done with the K / V buffers
    uint16_t* stage = &kbuf[0][0] + __builtin_amdgcn_readfirstlane(tx >> 6) * (32 * kBlock);
    const int col = tx & 31;
#pragma unroll
    for (int db = 0; db < 4; ++db) {
#pragma unroll
      for (int rr = 0; rr < 4; ++rr) {
        u32x2 v2;
        v2[0] = pack_bf16x2(ws.o[db][4 * rr] * inv, ws.o[db][4 * rr + 1] * inv);
        v2[1] = pack_bf16x2(ws.o[db][4 * rr + 2] * inv, ws.o[db][4 * rr + 3] * inv);
        const int c = db * 4 + rr;
        *reinterpret_cast<u32x2*>(stage + col * kBlock + ((c ^ (col & 15)) << 3) + 4 * half_e) = v2;
      }
    }
    const int lane = tx & 63;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int r = 4 * i + (lane >> 4), c = lane & 15;
      const u32x4 v4 = *reinterpret_cast<const u32x4*>(stage + r * kBlock + ((c ^ (r & 15)) << 3));
      const int64_t row = (int64_t)t * kBlock + wq * 32 + r;
      // non-temporal: the output is not read again here, and its lines would only
      // displace the K/V tiles the other items on this XCD are walking
      if (live && row < a.seq)
        __builtin_nontemporal_store(
            v4, reinterpret_cast<u32x4*>(static_cast<uint16_t*>(a.out) + b * a.os_b + row * a.os_s +
                                         h * a.os_h + c * 8));
    }
  }
  if (live && qrow < a.seq && a.lse && half_e == 0)
    a.lse[b * a.ls_b + qrow * a.ls_s + h * a.ls_h] = any ? ws.m * kLn2 + logf(l) : -INFINITY;
}

// ---------------------------------------------------------------- merge

struct MergeArgs {
  const uint16_t* eo;
  int64_t es_b, es_s, es_h;
  const float* el;
  int64_t els_b, els_s, els_h;
  const float* mo;
  int64_t ms_b, ms_s, ms_h;
  const float* ml;
  int64_t mls_b, mls_s, mls_h;
  uint16_t* out;
  int64_t os_b, os_s, os_h;
  float* lo;
  int64_t los_b, los_s, los_h;
  int batch, seq, heads, dim;
};

// One wave per (b, s, h) row of dim (128 or 256) dims; each lane handles 2 dims per
// 128.
__global__ __launch_bounds__(256) void merge_kernel(MergeArgs a) {
  const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  const int64_t rows = (int64_t)a.batch * a.seq * a.heads;
  if (row >= rows) return;
  const int h = row % a.heads;
  const int64_t s = (row / a.heads) % a.seq;
  const int b = row / ((int64_t)a.heads * a.seq);
  const int lane = threadIdx.x & 63;
  const float le = a.el[b * a.els_b + s * a.els_s + h * a.els_h];
  const float lm = a.ml[b * a.mls_b + s * a.mls_s + h * a.mls_h];
  // torch.logaddexp(a, b) = max + log1p(exp(-|a - b|)), -inf when both are -inf
  const float mx = fmaxf(le, lm);
  float total;
  if (mx == -INFINITY) total = -INFINITY;
  else if (le == lm) total = le + kLn2;
  else total = mx + log1pf(expf(-fabsf(le - lm)));
  const float we = expf(le - total);
  const float wm = expf(lm - total);
  for (int d = lane * 2; d < a.dim; d += 128) {
    const uint32_t e2 =
        *reinterpret_cast<const uint32_t*>(a.eo + b * a.es_b + s * a.es_s + h * a.es_h + d);
    const float* m2 = a.mo + b * a.ms_b + s * a.ms_s + h * a.ms_h + d;
    const float o0 = bf16_lo(e2) * we + m2[0] * wm;
    const float o1 = bf16_hi(e2) * we + m2[1] * wm;
    *reinterpret_cast<uint32_t*>(a.out + b * a.os_b + s * a.os_s + h * a.os_h + d) =
        pack_bf16x2(o0, o1);
  }
  if (a.lo && lane == 0) a.lo[b * a.los_b + s * a.los_s + h * a.los_h] = total;
}

}  // namespace spx

using namespace spx;

static int check_bsdh(const char* name, const void* p, const int64_t* st, bool need16) {
  SPX_REQUIRE(p != nullptr && st != nullptr, SPX_EINVAL, "%s: null pointer", name);
  SPX_REQUIRE(st[3] == 1, SPX_EINVAL, "%s: innermost (dim) stride must be 1", name);
  if (need16) {
    SPX_REQUIRE((reinterpret_cast<uintptr_t>(p) & 15) == 0, SPX_EINVAL,
                "%s: base pointer must be 16-byte aligned", name);
    SPX_REQUIRE(st[0] % 8 == 0 && st[1] % 8 == 0 && st[2] % 8 == 0, SPX_EINVAL,
                "%s: batch / sequence / head strides must be multiples of 8 elements", name);
  }
  return SPX_OK;
}

namespace {

struct AttnRequest {
  bool exact, tail, out_f32;
  int tail_kind;             // 0 block means, 1 rescue token, 2 rescue token + remainder
  const uint8_t* choice;     // rescue tokens (tail_kind > 0)
  const void* v;             // V rows of the rescue tokens (tail_kind > 0)
  const int64_t* v_strides;
  int32_t* work_queue;       // optional SPX_WORK_QUEUE_INTS zeroed int32: persistent grid
};

// Persistent grid: the last third of the tile pairs (the lightest: their lists are
// the shortest) form the shared tail.
constexpr int kStaticThirds = 2;

// Workgroups per XCD of the persistent grid: one per CU (the kernel's LDS and
// registers admit one workgroup per CU).
int persistent_per_xcd() {
  static int per_device[64] = {};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 32;
  if (per_device[dev] == 0) {
    int cus = 0;
    if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
        cus < 8)
      cus = 256;
    per_device[dev] = cus / 8;
  }
  return per_device[dev];
}

int launch_attention(const AttnRequest& req, const void* q, const int64_t* q_strides,
                     const void* key_tiles, const void* value_tiles,
                     const int64_t* indices, const int64_t* index_strides,
                     const int32_t* counts, const int64_t* count_strides,
                     const float* mean_k, const float* mean_v, const int32_t* block_counts,
                     int batch, int seq, int q_heads, int kv_heads, int head_dim,
                     int block_size, float scale, void* out, const int64_t* out_strides,
                     float* lse, const int64_t* lse_strides, void* stream) {
  SPX_REQUIRE(head_dim == kHeadDim || head_dim == 256, SPX_EUNSUPPORTED,
              "head_dim %d unsupported (128 or 256)", head_dim);
  SPX_REQUIRE(block_size == kBlock, SPX_EUNSUPPORTED, "block_size %d unsupported (only 128)", block_size);
  SPX_REQUIRE(batch > 0 && seq > 0 && q_heads > 0 && kv_heads > 0 && q_heads % kv_heads == 0,
              SPX_EINVAL, "bad shape: batch %d seq %d q_heads %d kv_heads %d", batch, seq,
              q_heads, kv_heads);
  const int blocks = num_blocks(seq);
  SPX_REQUIRE(blocks <= kMaxBlocksAttn, SPX_EUNSUPPORTED, "seq %d exceeds %d blocks", seq,
              kMaxBlocksAttn);
  int e = check_bsdh("q", q, q_strides, true);
  if (e) return e;
  e = check_bsdh("out", out, out_strides, true);
  if (e) return e;
  if (req.exact) {
    SPX_REQUIRE(key_tiles != nullptr && (reinterpret_cast<uintptr_t>(key_tiles) & 15) == 0,
                SPX_EINVAL, "key_tiles: null or not 16-byte aligned");
    SPX_REQUIRE(value_tiles != nullptr && (reinterpret_cast<uintptr_t>(value_tiles) & 15) == 0,
                SPX_EINVAL, "value_tiles: null or not 16-byte aligned");
  }
  if (req.tail && req.tail_kind == 0) {
    SPX_REQUIRE(mean_k && mean_v && block_counts, SPX_EINVAL,
                "mean correction needs mean_k, mean_v and block_counts");
  }
  if (req.tail && req.tail_kind > 0) {
    SPX_REQUIRE(req.choice != nullptr, SPX_EINVAL, "rescue tail needs the rescue token choice");
    SPX_REQUIRE(key_tiles != nullptr && (reinterpret_cast<uintptr_t>(key_tiles) & 15) == 0 &&
                    value_tiles != nullptr && (reinterpret_cast<uintptr_t>(value_tiles) & 15) == 0,
                SPX_EINVAL, "rescue tail needs 16-byte aligned key_tiles and value_tiles");
    SPX_REQUIRE(req.tail_kind == 1 || (mean_k && mean_v), SPX_EINVAL,
                "rescue remainder needs mean_k and mean_v");
    int ev = check_bsdh("v", req.v, req.v_strides, true);
    if (ev) return ev;
  }
  if (indices) {
    SPX_REQUIRE(index_strides && counts && count_strides, SPX_EINVAL,
                "indices given without strides / counts");
  } else {
    SPX_REQUIRE(req.exact, SPX_EINVAL, "mean_tail needs index lists");
  }
  if (lse) SPX_REQUIRE(lse_strides != nullptr, SPX_EINVAL, "lse strides missing");
  if (head_dim == 256) {
    const Attn256Options opt{req.exact, req.tail, req.out_f32, req.tail_kind, mean_k, mean_v,
                             block_counts, req.choice, req.v, req.v_strides, req.work_queue};
    return launch_attention_256(opt, q, q_strides, key_tiles, value_tiles, indices, index_strides,
                                counts, count_strides, batch, seq, q_heads, kv_heads, scale, out,
                                out_strides, lse, lse_strides, stream);
  }

  AttnArgs a{};
  a.q = static_cast<const uint16_t*>(q);
  a.qs_b = q_strides[0]; a.qs_s = q_strides[1]; a.qs_h = q_strides[2];
  a.kt = static_cast<const uint16_t*>(key_tiles);
  a.vt = static_cast<const uint16_t*>(value_tiles);
  a.idx = indices;
  if (indices) {
    a.is_b = index_strides[0]; a.is_t = index_strides[1]; a.is_p = index_strides[2];
    a.is_h = index_strides[3];
    a.cnt = counts;
    a.cs_b = count_strides[0]; a.cs_t = count_strides[1]; a.cs_h = count_strides[2];
  }
  a.mean_k = mean_k; a.mean_v = mean_v; a.bcounts = block_counts;
  a.choice = req.choice; a.tail_kind = req.tail ? req.tail_kind : 0;
  if (req.tail && req.tail_kind > 0) {
    a.v = static_cast<const uint16_t*>(req.v);
    a.vs_b = req.v_strides[0]; a.vs_s = req.v_strides[1]; a.vs_h = req.v_strides[2];
  }
  a.out = out;
  a.os_b = out_strides[0]; a.os_s = out_strides[1]; a.os_h = out_strides[2];
  a.lse = lse;
  if (lse) { a.ls_b = lse_strides[0]; a.ls_s = lse_strides[1]; a.ls_h = lse_strides[2]; }
  a.batch = batch; a.seq = seq; a.q_heads = q_heads; a.kv_heads = kv_heads;
  a.blocks = blocks; a.group = q_heads / kv_heads;
  a.num_pairs = ((blocks + 1) / 2) * batch * kv_heads;  // (tile pair, batch, kv group)
  a.scale_log2 = (float)((double)scale * 1.4426950408889634);
  const int streams = batch * kv_heads;
  a.xcds_per_stream = (streams <= 8 && 8 % streams == 0) ? 8 / streams : 1;
  const int np = (blocks + 1) / 2;
  const int per_xcd = a.xcds_per_stream > 1
      ? (np * a.group + a.xcds_per_stream - 1) / a.xcds_per_stream
      : (a.num_pairs + 7) / 8 * a.group;
  a.static_tp = np;
  int grid = 8 * per_xcd;
  if (req.work_queue) {
    SPX_REQUIRE((reinterpret_cast<uintptr_t>(req.work_queue) & 3) == 0, SPX_EINVAL,
                "work_queue must be 4-byte aligned");
    int tp0 = np * kStaticThirds / 3;
    while (tp0 > 0 && a.xcds_per_stream > 1 && (tp0 * a.group) % a.xcds_per_stream) --tp0;
    a.queue = req.work_queue;
    a.static_tp = tp0;
    a.dyn_items = (np - tp0) * streams * a.group;
    grid = 8 * std::min(persistent_per_xcd(), per_xcd);
  }
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (req.exact && !req.tail) attn_kernel<true, false, false><<<grid, kAttnThreads, 0, st>>>(a);
  else if (req.exact && req.tail) attn_kernel<true, true, false><<<grid, kAttnThreads, 0, st>>>(a);
  else attn_kernel<false, true, true><<<grid, kAttnThreads, 0, st>>>(a);
  return launch_status("attention");
}

}  // namespace

extern "C" int spx_exact_attention(const void* q, const int64_t* q_strides,
                                   const void* key_tiles, const void* value_tiles,
                                   const int64_t* indices, const int64_t* index_strides,
                                   const int32_t* counts, const int64_t* count_strides, int batch,
                                   int seq, int q_heads, int kv_heads, int head_dim,
                                   int block_size, float scale, void* out,
                                   const int64_t* out_strides, float* lse,
                                   const int64_t* lse_strides, int32_t* work_queue, void* stream) {
  return launch_attention({true, false, false, 0, nullptr, nullptr, nullptr, work_queue}, q, q_strides, key_tiles, value_tiles, indices,
                          index_strides, counts, count_strides, nullptr, nullptr, nullptr, batch,
                          seq, q_heads, kv_heads, head_dim, block_size, scale, out, out_strides,
                          lse, lse_strides, stream);
}

extern "C" int spx_sparse_attention_mean(const void* q, const int64_t* q_strides,
                                         const void* key_tiles, const void* value_tiles,
                                         const int64_t* indices, const int64_t* index_strides,
                                         const int32_t* counts, const int64_t* count_strides,
                                         const float* mean_k, const float* mean_v,
                                         const int32_t* block_counts, int batch, int seq,
                                         int q_heads, int kv_heads, int head_dim, int block_size,
                                         float scale, void* out, const int64_t* out_strides,
                                         float* lse, const int64_t* lse_strides,
                                         int32_t* work_queue, void* stream) {
  return launch_attention({true, true, false, 0, nullptr, nullptr, nullptr, work_queue}, q, q_strides, key_tiles, value_tiles, indices,
                          index_strides, counts, count_strides, mean_k, mean_v, block_counts,
                          batch, seq, q_heads, kv_heads, head_dim, block_size, scale, out,
                          out_strides, lse, lse_strides, stream);
}

extern "C" int spx_mean_tail(const void* q, const int64_t* q_strides, const int64_t* indices,
                             const int64_t* index_strides, const int32_t* counts,
                             const int64_t* count_strides, const float* mean_k,
                             const float* mean_v, const int32_t* block_counts, int batch, int seq,
                             int q_heads, int kv_heads, int head_dim, int block_size, float scale,
                             float* out, const int64_t* out_strides, float* lse,
                             const int64_t* lse_strides, void* stream) {
  SPX_REQUIRE(indices != nullptr, SPX_EINVAL, "mean_tail: indices must be given");
  return launch_attention({false, true, true, 0, nullptr}, q, q_strides, nullptr, nullptr, indices,
                          index_strides, counts, count_strides, mean_k, mean_v, block_counts,
                          batch, seq, q_heads, kv_heads, head_dim, block_size, scale, out,
                          out_strides, lse, lse_strides, stream);
}

extern "C" int spx_merge_exact_mean(const void* exact_out, const int64_t* exact_strides,
                                    const float* exact_lse, const int64_t* exact_lse_strides,
                                    const float* mean_out, const int64_t* mean_strides,
                                    const float* mean_lse, const int64_t* mean_lse_strides,
                                    int batch, int seq, int heads, int head_dim, void* out,
                                    const int64_t* out_strides, float* lse_out,
                                    const int64_t* lse_out_strides, void* stream) {
  SPX_REQUIRE(head_dim == kHeadDim || head_dim == 256, SPX_EUNSUPPORTED,
              "head_dim %d unsupported (128 or 256)", head_dim);
  SPX_REQUIRE(batch > 0 && seq > 0 && heads > 0, SPX_EINVAL, "bad shape");
  int e = check_bsdh("exact_out", exact_out, exact_strides, false);
  if (e) return e;
  e = check_bsdh("mean_out", mean_out, mean_strides, false);
  if (e) return e;
  e = check_bsdh("out", out, out_strides, false);
  if (e) return e;
  SPX_REQUIRE(exact_lse && exact_lse_strides && mean_lse && mean_lse_strides, SPX_EINVAL,
              "lse inputs missing");
  SPX_REQUIRE(exact_strides[0] % 2 == 0 && exact_strides[1] % 2 == 0 && exact_strides[2] % 2 == 0 &&
              out_strides[0] % 2 == 0 && out_strides[1] % 2 == 0 && out_strides[2] % 2 == 0,
              SPX_EINVAL, "bf16 strides must be even");
  MergeArgs a{};
  a.eo = static_cast<const uint16_t*>(exact_out);
  a.es_b = exact_strides[0]; a.es_s = exact_strides[1]; a.es_h = exact_strides[2];
  a.el = exact_lse;
  a.els_b = exact_lse_strides[0]; a.els_s = exact_lse_strides[1]; a.els_h = exact_lse_strides[2];
  a.mo = mean_out;
  a.ms_b = mean_strides[0]; a.ms_s = mean_strides[1]; a.ms_h = mean_strides[2];
  a.ml = mean_lse;
  a.mls_b = mean_lse_strides[0]; a.mls_s = mean_lse_strides[1]; a.mls_h = mean_lse_strides[2];
  a.out = static_cast<uint16_t*>(out);
  a.os_b = out_strides[0]; a.os_s = out_strides[1]; a.os_h = out_strides[2];
  a.lo = lse_out;
  if (lse_out) {
    SPX_REQUIRE(lse_out_strides != nullptr, SPX_EINVAL, "lse_out strides missing");
    a.los_b = lse_out_strides[0]; a.los_s = lse_out_strides[1]; a.los_h = lse_out_strides[2];
  }
  a.batch = batch; a.seq = seq; a.heads = heads; a.dim = head_dim;
  const int64_t rows = (int64_t)batch * seq * heads;
  const int grid = (int)((rows + 3) / 4);
  merge_kernel<<<grid, 256, 0, static_cast<hipStream_t>(stream)>>>(a);
  return launch_status("merge_exact_mean");
}

extern "C" int spx_sparse_attention_rescue(
    const void* q, const int64_t* q_strides, const void* key_tiles, const void* value_tiles,
    const int64_t* indices, const int64_t* index_strides, const int32_t* counts,
    const int64_t* count_strides, const uint8_t* choice, const void* v, const int64_t* v_strides,
    const float* mean_k, const float* mean_v, int remainder, int batch, int seq, int q_heads,
    int kv_heads, int head_dim, int block_size, float scale, void* out, const int64_t* out_strides,
    float* lse, const int64_t* lse_strides, int32_t* work_queue, void* stream) {
  return launch_attention({true, true, false, remainder ? 2 : 1, choice, v, v_strides, work_queue}, q, q_strides,
                          key_tiles,
                          value_tiles, indices, index_strides, counts, count_strides, mean_k,
                          mean_v, nullptr, batch, seq, q_heads, kv_heads, head_dim, block_size,
                          scale, out, out_strides, lse, lse_strides, stream);
}

extern "C" int spx_rescue_tail(const void* q, const int64_t* q_strides, const void* key_tiles,
                               const void* value_tiles, const int64_t* indices,
                               const int64_t* index_strides, const int32_t* counts,
                               const int64_t* count_strides, const uint8_t* choice,
                               const void* v, const int64_t* v_strides, const float* mean_k,
                               const float* mean_v, int remainder, int batch, int seq, int q_heads,
                               int kv_heads, int head_dim, int block_size, float scale, float* out,
                               const int64_t* out_strides, float* lse, const int64_t* lse_strides,
                               void* stream) {
  SPX_REQUIRE(indices != nullptr, SPX_EINVAL, "rescue_tail: indices must be given");
  return launch_attention({false, true, true, remainder ? 2 : 1, choice, v, v_strides}, q, q_strides,
                          key_tiles,
                          value_tiles, indices, index_strides, counts, count_strides, mean_k,
                          mean_v, nullptr, batch, seq, q_heads, kv_heads, head_dim, block_size,
                          scale, out, out_strides, lse, lse_strides, stream);
}

