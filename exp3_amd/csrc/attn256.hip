// Block-sparse causal flash attention at head_dim 256 (Qwen3.5 full-attention
// layers, 16:4 GQA; check_qwen35_math.py; upstream/flashprefill_native_forward.py
// :215-354 / :478-521 with D = 256, whose Triton launch walks each 128-token block
// in four 32-key micro-tiles).
//
// gfx950 mapping
//   * One workgroup per (query tile t, q head h): four waves of 32 query rows, one
//     wave per SIMD. A wave keeps its Q rows in registers as MFMA B operands (16
//     k-steps of 16 dims) and O^T (256 dims x 32 queries, eight 32 x 32 tiles) in
//     the accumulators.
//   * Keys stream in 32-key sub-blocks: the K rows (16 KB) and V^T (256 dims x 32
//     key slots, 16 KB) of a sub-block are contiguous in the pool's d = 256 tiles and
//     are copied verbatim into one of two LDS buffer pairs with direct global->LDS
//     loads while the previous sub-block is computed (one barrier per sub-block).
//   * Scores are formed transposed, S^T = K Q^T (v_mfma_f32_32x32x16_bf16, 16
//     k-steps), so each lane owns one query column: the online softmax is in-lane
//     plus one lane-half exchange, and the probabilities already sit in the B-operand
//     layout of O^T += V^T P^T (key slot permutation of the value tiles). The running
//     max moves only when a column's shifted score x = s * scale - m exceeds 2^64
//     (lazy rescale); the common path checks each lane half's own max of x.
//   * The tile's list (entries outside [0, NB) skipped, as the reference's loop
//     never reads them usefully) is compacted into LDS once; as in the reference,
//     only the diagonal block j == t is masked (key > query).
//   * Tails (mean methods, kernels.py:179-230 + :312-325; rescue methods,
//     kernels.py:233-309), after the exact blocks inside the same online softmax:
//     the history blocks j < t the tile does not list, 32 entries per sub-block,
//     staged into LDS by all four waves. An entry's key is an fp32 vector (block
//     mean, or (128 mean - token) / 127 for the rescue remainder) split into bf16
//     hi and lo rows in the two K buffers, whose products are summed (fp32-accurate
//     logits); its value is bf16 in the first V buffer; its logit bias (ln n_j, 0 or
//     ln 127) is added after scaling. Exact keys (rescue tokens) have lo rows 0.
#include "common.h"

namespace spx {

constexpr int kD2 = 256;
constexpr int kSub = 32;                   // keys per sub-block
constexpr int kSubElems = kSub * kD2;      // 8192 bf16 = 16 KB
constexpr int kA2Threads = 256;
constexpr int kA2MaxBlocks = 1024;
constexpr float kLazy = 64.0f;             // log2 headroom before a column's running max moves
                                           // (bf16 P, fp32 O and l: 2^64 loses nothing)

struct Attn256Args {
  const uint16_t* q;
  int64_t qs_b, qs_s, qs_h;
  const uint16_t* kt;  // [B, Hkv, NB, 128, 256]: K rows, chunk c of row r at c ^ (r & 15)
  const uint16_t* vt;  // [B, Hkv, NB, 4, 256, 32]: V^T per sub-block, chunk c of row d at c ^ ((d >> 2) & 3)
  const int64_t* idx;  // [B, NB, NB, Hq] (strided) or null for every causal block
  int64_t is_b, is_t, is_p, is_h;
  const int32_t* cnt;
  int64_t cs_b, cs_t, cs_h;
  int batch, seq, q_heads, kv_heads, blocks;
  float scale_log2;
  void* out;           // bf16, or fp32 for the tail-only entry points
  int64_t os_b, os_s, os_h;
  float* lse;
  int64_t ls_b, ls_s, ls_h;
  // tails
  int tail_kind;       // 0 block means, 1 rescue token, 2 rescue token + remainder
  const float* mean_k; // [B, NB, Hkv, 256]
  const float* mean_v;
  const int32_t* bcounts;
  const uint8_t* choice;
  const uint16_t* v;
  int64_t vs_b, vs_s, vs_h;
  // dynamic tail: tile ranks >= static_ranks are taken from a zeroed counter
  int* queue;          // null: every workgroup on the static grid
  int static_ranks;
  int dyn_items;
};

// Position of 16-byte chunk c (< 32) of K row r in the d = 256 key layout.
__device__ __forceinline__ int key_chunk_pos(int r, int c) { return (c & 16) | ((c & 15) ^ (r & 15)); }

// The rare branch of the lazy max and the probability / P V half of a 32-key
// sub-block, on shifted scores x = s * scale (+ bias) - m (masked keys -inf).
__device__ __forceinline__ void softmax_pv(f32x16& x, const uint16_t* vb, f32x16 (&o)[8],
                                           float& neg_m, float& thr, float& l) {
  const int lane = threadIdx.x & 63;
  const int col = lane & 31, half = lane >> 5;
  const int vsw = (col >> 2) & 3;
  float mx = fmaxf(fmaxf(x[0], x[1]), x[2]);
#pragma unroll
  for (int r = 3; r < 15; r += 2) mx = fmaxf(fmaxf(mx, x[r]), x[r + 1]);
  mx = fmaxf(mx, x[15]);
  if (__any(mx > thr)) {
    const auto sw = __builtin_amdgcn_permlane32_swap(__float_as_uint(mx), __float_as_uint(mx),
                                                     false, false);
    mx = fmaxf(__uint_as_float(sw[0]), __uint_as_float(sw[1]));
    const bool move = mx > thr;
    const float d = move ? mx : 0.0f;
    // nothing is accumulated before the first move (thr -inf): O and l stay 0
    const float corr = thr == -INFINITY ? 0.0f : exp2_fast(-d);
    // in place (tied operands): O keeps its registers across the rare branch. The
    // compiler's hazard recognizer does not look inside asm statements, so the
    // wait states after the last product into O (19 >= the XDL write -> VALU
    // requirement) are issued first, tied to O.
    asm volatile("s_nop 7\n\ts_nop 7\n\ts_nop 2"
                 : "+v"(o[0]), "+v"(o[1]), "+v"(o[2]), "+v"(o[3]), "+v"(o[4]), "+v"(o[5]),
                   "+v"(o[6]), "+v"(o[7]));
#pragma unroll
    for (int dt = 0; dt < 8; ++dt)
#pragma unroll
      for (int r = 0; r < 16; ++r) asm volatile("v_mul_f32 %0, %0, %1" : "+v"(o[dt][r]) : "v"(corr));
    l *= corr;
    neg_m -= d;
    if (move) thr = kLazy;
#pragma unroll
    for (int r = 0; r < 16; ++r) x[r] -= d;
  }
  // probabilities as bf16 B operands; the running sum adds the fp32 probabilities
  // (upstream/flashprefill_native_forward.py:332-338), pairwise: plain adds run
  // beside the matrix products almost for free, v_dot2_f32_bf16 sums of the packed
  // pairs did not
  u32x4 pb0, pb1;
  float pair_sum[8];
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    const float a0 = exp2_fast(x[2 * e]), b0 = exp2_fast(x[2 * e + 1]);
    const float a1 = exp2_fast(x[8 + 2 * e]), b1 = exp2_fast(x[8 + 2 * e + 1]);
    pb0[e] = pack_bf16x2(a0, b0);
    pb1[e] = pack_bf16x2(a1, b1);
    pair_sum[e] = a0 + b0;
    pair_sum[4 + e] = a1 + b1;
  }
  l += ((pair_sum[0] + pair_sum[1]) + (pair_sum[2] + pair_sum[3])) +
       ((pair_sum[4] + pair_sum[5]) + (pair_sum[6] + pair_sum[7]));
#pragma unroll
  for (int d2 = 0; d2 < 4; ++d2) {
    bf16x8 vr[4];
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const uint16_t* vrow = vb + ((2 * d2 + i) * 32 + col) * kSub;
      vr[2 * i] = as_bf16x8(*reinterpret_cast<const u32x4*>(vrow + ((half ^ vsw) << 3)));
      vr[2 * i + 1] =
          as_bf16x8(*reinterpret_cast<const u32x4*>(vrow + (((2 + half) ^ vsw) << 3)));
    }
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      o[2 * d2 + i] = mfma32(vr[2 * i], as_bf16x8(pb0), o[2 * d2 + i]);
      o[2 * d2 + i] = mfma32(vr[2 * i + 1], as_bf16x8(pb1), o[2 * d2 + i]);
    }
    __builtin_amdgcn_sched_barrier(0);
  }
}

// S^T += K Q^T over the 16 k-steps of one 32-row K buffer; operand reads in groups
// of four k-steps (fenced), so that at most four K operands are live: with O (128)
// and Q (64) the wave stays under 256 VGPRs and O never leaves its registers.
__device__ __forceinline__ void key_products(const uint16_t* kb, int e0, const bf16x8 (&qb)[16],
                                             f32x16& sc) {
#pragma unroll
  for (int g4 = 0; g4 < 4; ++g4) {
    bf16x8 kr[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int dc = g4 * 4 + i;
      kr[i] = as_bf16x8(*reinterpret_cast<const u32x4*>(kb + (dc >> 3) * 128 +
                                                          (e0 ^ ((dc & 7) << 4))));
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) sc = mfma32(kr[i], qb[g4 * 4 + i], sc);
    __builtin_amdgcn_sched_barrier(0);
  }
}

// Tail sub-block entry i (< 32), 8-dim chunk c (< 32): key hi / lo rows in kh / kl,
// value in slot value_slot_of_key(i) of dim rows 8c .. 8c + 7 of vb.
__device__ __forceinline__ void write_tail_entry256(uint16_t* kh, uint16_t* kl, uint16_t* vb,
                                                   int i, int c, const float (&mk)[8],
                                                   const float (&mv)[8]) {
  u32x4 hi, lo;
#pragma unroll
  for (int x = 0; x < 4; ++x) {
    const uint32_t h2 = pack_bf16x2(mk[2 * x], mk[2 * x + 1]);
    hi[x] = h2;
    lo[x] = pack_bf16x2(mk[2 * x] - bf16_lo(h2), mk[2 * x + 1] - bf16_hi(h2));
  }
  const int koff = i * kD2 + key_chunk_pos(i, c) * 8;
  *reinterpret_cast<u32x4*>(kh + koff) = hi;
  *reinterpret_cast<u32x4*>(kl + koff) = lo;
  const int slot = value_slot_of_key(i);
#pragma unroll
  for (int x = 0; x < 8; ++x) {
    const int d = c * 8 + x;
    vb[d * kSub + ((((slot >> 3) ^ ((d >> 2) & 3))) << 3) + (slot & 7)] = to_bf16_bits(mv[x]);
  }
}

// 16 KB from global memory into LDS: four instructions of 256 lanes x 16 bytes.
__device__ __forceinline__ void dma_16k(const uint16_t* src, uint16_t* lds, int tid) {
  const int w = tid >> 6;
  const uint32_t lds_base =
      (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) uint16_t*)lds;
  const uint32_t voff = (uint32_t)tid * 16u;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const uint32_t m0 =
        __builtin_amdgcn_readfirstlane(lds_base + (uint32_t)(i * kA2Threads + w * 64) * 16u);
    const uint16_t* s = src + i * kA2Threads * 8;
    uint32_t saved;
    asm volatile(
        "s_mov_b32 %0, m0\n\t"
        "s_mov_b32 m0, %1\n\t"
        "s_nop 0\n\t"
        "global_load_lds_dwordx4 %2, %3\n\t"
        "s_mov_b32 m0, %0"
        : "=&s"(saved)
        : "s"(m0), "v"(voff), "s"(s)
        : "memory");
  }
}

template <bool EXACT, bool TAIL, bool OUT_F32>
__global__ __launch_bounds__(kA2Threads, 1) void attn256_kernel(Attn256Args a) {
  const int per_tile = a.batch * a.q_heads;
  int rank = (int)(blockIdx.x / per_tile), bh = (int)(blockIdx.x % per_tile);
  if (a.queue && rank >= a.static_ranks) {
    // dynamic tail: XCDs run at different speeds and workgroup i is bound to XCD
    // i % 8, so the light tiles go to whichever workgroups run first (surplus ones
    // find the counter past the end and exit)
    __shared__ int dyn_k;
    if (threadIdx.x == 0) dyn_k = atomicAdd(a.queue, 1);
    block_sync();
    const int kd = dyn_k;
    if (kd >= a.dyn_items) return;
    rank = a.static_ranks + kd / per_tile;
    bh = kd % per_tile;
  }
  const int t = a.blocks - 1 - rank;  // heaviest tiles first
  const int b = bh / a.q_heads, h = bh % a.q_heads;
  const int g = h / (a.q_heads / a.kv_heads);
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int col = lane & 31, half = lane >> 5;

  __shared__ __align__(16) uint16_t kbuf[2][kSubElems];
  __shared__ __align__(16) uint16_t vbuf[2][kSubElems];
  __shared__ int list[kA2MaxBlocks];
  __shared__ int list_len;
  __shared__ uint32_t listed[TAIL ? kA2MaxBlocks / 32 : 1];   // membership of the tile's list
  __shared__ int16_t tlist[TAIL ? kA2MaxBlocks : 1];          // unlisted history blocks
  __shared__ float tail_bias[kSub];
  __shared__ int tail_len;

  if (TAIL) {
    if (tid < kA2MaxBlocks / 32) listed[tid] = 0u;
    block_sync();
  }
  // compacted block list: ids in [0, NB), list order
  if (w == 0) {
    int n = a.idx ? a.cnt[b * a.cs_b + t * a.cs_t + h * a.cs_h] : t + 1;
    n = max(0, min(n, a.blocks));
    int base = 0;
    for (int u0 = 0; u0 < n; u0 += 64) {
      const int u = u0 + lane;
      int64_t j = -1;   // range-checked before narrowing
      if (u < n) j = a.idx ? a.idx[b * a.is_b + t * a.is_t + u * a.is_p + h * a.is_h] : u;
      const bool ok = j >= 0 && j < a.blocks;
      const uint64_t m = __ballot(ok);
      const int pos = base + __popcll(m & ((1ull << lane) - 1ull));
      if (ok) {
        list[pos] = (int)j;
        if (TAIL) atomicOr(&listed[j >> 5], 1u << (j & 31));
      }
      base += __popcll(m);
    }
    if (lane == 0) list_len = base;
  }
  block_sync();
  const int steps = EXACT ? list_len * 4 : 0;
  const int64_t kv_block0 = ((int64_t)b * a.kv_heads + g) * a.blocks;

  auto issue = [&](int s, int buf) {
    const int j = __builtin_amdgcn_readfirstlane(list[s >> 2]);
    const int sb = s & 3;
    dma_16k(a.kt + ((kv_block0 + j) * kBlock + sb * kSub) * kD2, kbuf[buf], tid);
    dma_16k(a.vt + (kv_block0 + j) * (kBlock * kD2) + sb * kSubElems, vbuf[buf], tid);
  };
  if (steps > 0) issue(0, 0);

  const int qr = w * 32 + col;  // query row within the tile
  const int64_t qrow = (int64_t)t * kBlock + qr;
  const bool row_ok = qrow < a.seq;
  bf16x8 qb[16];
  {
    const uint16_t* src = a.q + b * a.qs_b + qrow * a.qs_s + h * a.qs_h + half * 8;
#pragma unroll
    for (int dc = 0; dc < 16; ++dc) {
      u32x4 raw = {0u, 0u, 0u, 0u};
      if (row_ok) raw = *reinterpret_cast<const u32x4*>(src + dc * 16);
      asm volatile("" : "+v"(raw));  // consume now: its wait stays outside the loop
      qb[dc] = as_bf16x8(raw);
    }
  }

  // K operand: row col, 16-byte chunk 2 dc + half at ((2 dc + half) ^ (col & 15)):
  // (dc >> 3) * 128 + (e0 ^ ((dc & 7) << 4)) elements past the row start.
  const int e0 = (((col >> 1) & 7) << 4) + ((half ^ (col & 1)) << 3);

  f32x16 o[8];
#pragma unroll
  for (int dt = 0; dt < 8; ++dt) o[dt] = f32x16{};
  float neg_m = 0.0f;        // -(running max) in log2 units once set (0 before)
  float thr = -INFINITY;     // lazy-move threshold on shifted scores (-inf before the max is set)
  float l = 0.0f;            // this half's share of the probability sum

  for (int s = 0; s < steps; ++s) {
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    block_sync();  // sub-block s landed everywhere; buffers (s + 1) & 1 are free
    if (s + 1 < steps) issue(s + 1, (s + 1) & 1);
    const int j = __builtin_amdgcn_readfirstlane(list[s >> 2]);
    const int sb = s & 3;
    f32x16 sc = {};
    key_products(kbuf[s & 1] + col * kD2, e0, qb, sc);
    // x = s * scale - m (diagonal block: keys above the query at -inf); the lazy
    // max check runs on x, per lane half, and forms the column max over both
    // halves only in the rare branch where some lane exceeds its threshold
    f32x16 x;
#pragma unroll
    for (int r = 0; r < 16; ++r) x[r] = fmaf(sc[r], a.scale_log2, neg_m);
    if (j == t) {
#pragma unroll
      for (int r = 0; r < 16; ++r)
        if (sb * kSub + mfma32_row(r, lane) > qr) x[r] = -INFINITY;
    }
    softmax_pv(x, vbuf[s & 1], o, neg_m, thr, l);
  }

  if constexpr (TAIL) {
    // the tail: history blocks j < t the tile does not list, ascending
    if (w == 0) {
      int base = 0;
      for (int j0 = 0; j0 < t; j0 += 64) {
        const int j = j0 + lane;
        const bool in = j < t && !((listed[j >> 5] >> (j & 31)) & 1u);
        const uint64_t m = __ballot(in);
        if (in) tlist[base + __popcll(m & ((1ull << lane) - 1ull))] = (int16_t)j;
        base += __popcll(m);
      }
      if (lane == 0) tail_len = base;
    }
    block_sync();  // also: every wave is done with the exact blocks' buffers
    const int ntail = tail_len;
    const int epb = a.tail_kind == 2 ? 2 : 1;  // entries per unlisted block
    const int per_sub = kSub / epb;
    for (int t0 = 0; t0 < ntail; t0 += per_sub) {
      if (t0 > 0) block_sync();  // every wave is done with the previous tail sub-block
      // one work item per (entry, 8-dim chunk): 32 x 32 over the four waves. Not
      // unrolled: with O (128) and Q (64) live, four items' temporaries at once
      // would push the wave past 256 registers (AGPR spills, one wave per SIMD)
#pragma unroll 1
      for (int k4 = 0; k4 < (kSub * (kD2 / 8)) / kA2Threads; ++k4) {
        const int e = opaque(tid) + k4 * kA2Threads;
        const int i = e >> 5, c = e & 31;
        const int blk = t0 + i / epb, kind = i % epb;
        const int j = blk < ntail ? (int)tlist[blk] : -1;
        float mk[8] = {}, mv[8] = {};
        float bi = -INFINITY;
        if (j >= 0) {
          const int64_t off = (((int64_t)b * a.blocks + j) * a.kv_heads + g) * kD2 + c * 8;
          if (a.tail_kind == 0) {
            load8(a.mean_k + off, mk);
            load8(a.mean_v + off, mv);
            bi = logf((float)a.bcounts[j]) * kLog2e;
          } else {
            // history blocks j < t are full, so the token is inside the sequence
            const int tok = a.choice[(((int64_t)b * a.blocks + t) * a.blocks + j) * a.q_heads + h];
            const u32x4 kraw = *reinterpret_cast<const u32x4*>(
                a.kt + ((kv_block0 + j) * kBlock + tok) * kD2 + key_chunk_pos(tok, c) * 8);
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
        }
        write_tail_entry256(kbuf[0], kbuf[1], vbuf[0], i, c, mk, mv);
        if (c == 0) tail_bias[i] = bi;
      }
      block_sync();
      const int lane_t = opaque(lane);
      const int col_t = lane_t & 31;
      const int e0_t = (((col_t >> 1) & 7) << 4) + (((lane_t >> 5) ^ (col_t & 1)) << 3);
      f32x16 sc = {};
      key_products(kbuf[0] + col_t * kD2, e0_t, qb, sc);   // hi rows
      key_products(kbuf[1] + col_t * kD2, e0_t, qb, sc);   // lo rows
      f32x16 x;
#pragma unroll
      for (int r = 0; r < 16; ++r)
        x[r] = fmaf(sc[r], a.scale_log2, tail_bias[mfma32_row(r, lane_t)]) + neg_m;
      softmax_pv(x, vbuf[0], o, neg_m, thr, l);
    }
  }

  l += __shfl_xor(l, 32);
  const float inv = l > 0.0f ? 1.0f / l : 0.0f;
  if (OUT_F32) {
    if (row_ok) {
      float* dst = static_cast<float*>(a.out) + b * a.os_b + qrow * a.os_s + h * a.os_h + 4 * half;
#pragma unroll
      for (int dt = 0; dt < 8; ++dt) {
#pragma unroll
        for (int grp = 0; grp < 4; ++grp) {
          const int r = 4 * grp;
          *reinterpret_cast<f32x4*>(dst + dt * 32 + 8 * grp) =
              f32x4{o[dt][r] * inv, o[dt][r + 1] * inv, o[dt][r + 2] * inv, o[dt][r + 3] * inv};
        }
      }
    }
  } else {
    // Each lane holds 4-dim pieces of its query row, so stored directly every store
    // instruction would write 16 bytes into each of 32 rows. The wave stages its
    // 32 x 256 bf16 rows in one of the (now free) K / V buffers, 16-byte chunk c of
    // row r at c ^ (r & 31), and stores whole 512-byte rows, 32 lanes per row.
    block_sync();   // every wave is done with the K / V buffers
    // lane values re-derived here, so that nothing computed from them is hoisted
    // above the block loops and held there
    const int tx = opaque((int)threadIdx.x);
    const int wv = __builtin_amdgcn_readfirstlane(tx >> 6);
    const int lane_e = tx & 63, col_e = tx & 31, half_e = (tx >> 5) & 1;
    uint16_t* stage = wv < 2 ? kbuf[wv] : vbuf[wv - 2];
#pragma unroll
    for (int dt = 0; dt < 8; ++dt) {
#pragma unroll
      for (int grp = 0; grp < 4; ++grp) {
        const int r = 4 * grp;
        u32x2 v;
        v[0] = pack_bf16x2(o[dt][r] * inv, o[dt][r + 1] * inv);
        v[1] = pack_bf16x2(o[dt][r + 2] * inv, o[dt][r + 3] * inv);
        const int c = dt * 4 + grp;
        *reinterpret_cast<u32x2*>(stage + col_e * kD2 + ((c ^ col_e) << 3) + 4 * half_e) = v;
      }
    }
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const int r = 2 * i + (lane_e >> 5), c = lane_e & 31;
      const u32x4 v4 = *reinterpret_cast<const u32x4*>(stage + r * kD2 + ((c ^ r) << 3));
      const int64_t row = (int64_t)t * kBlock + wv * 32 + r;
      if (row < a.seq)   // non-temporal: not read again here (keeps the K/V sub-blocks in L2)
        __builtin_nontemporal_store(
            v4, reinterpret_cast<u32x4*>(static_cast<uint16_t*>(a.out) + b * a.os_b + row * a.os_s +
                                         h * a.os_h + c * 8));
    }
  }
  if (row_ok && a.lse && half == 0)
    a.lse[b * a.ls_b + qrow * a.ls_s + h * a.ls_h] =
        l > 0.0f ? (log2f(l) - neg_m) * kLn2 : -INFINITY;
}

int launch_attention_256(const Attn256Options& opt, const void* q, const int64_t* q_strides,
                         const void* key_tiles, const void* value_tiles, const int64_t* indices,
                         const int64_t* index_strides, const int32_t* counts,
                         const int64_t* count_strides, int batch, int seq, int q_heads,
                         int kv_heads, float scale, void* out, const int64_t* out_strides,
                         float* lse, const int64_t* lse_strides, void* stream) {
  const int blocks = num_blocks(seq);
  SPX_REQUIRE(blocks <= kA2MaxBlocks, SPX_EUNSUPPORTED, "seq %d exceeds %d blocks", seq,
              kA2MaxBlocks);
  Attn256Args a{};
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
  a.batch = batch; a.seq = seq; a.q_heads = q_heads; a.kv_heads = kv_heads; a.blocks = blocks;
  a.scale_log2 = (float)((double)scale * 1.4426950408889634);
  a.out = out;
  a.os_b = out_strides[0]; a.os_s = out_strides[1]; a.os_h = out_strides[2];
  a.lse = lse;
  if (lse) { a.ls_b = lse_strides[0]; a.ls_s = lse_strides[1]; a.ls_h = lse_strides[2]; }
  if (opt.tail) {
    a.tail_kind = opt.tail_kind;
    a.mean_k = opt.mean_k; a.mean_v = opt.mean_v; a.bcounts = opt.block_counts;
    a.choice = opt.choice;
    if (opt.tail_kind > 0) {
      a.v = static_cast<const uint16_t*>(opt.v);
      a.vs_b = opt.v_strides[0]; a.vs_s = opt.v_strides[1]; a.vs_h = opt.v_strides[2];
    }
  }
  unsigned grid = (unsigned)(blocks * batch * q_heads);
  if (opt.work_queue) {
    SPX_REQUIRE((reinterpret_cast<uintptr_t>(opt.work_queue) & 3) == 0, SPX_EINVAL,
                "work_queue must be 4-byte aligned");
    a.queue = opt.work_queue;
    a.static_ranks = blocks * 2 / 3;
    a.dyn_items = (blocks - a.static_ranks) * batch * q_heads;
    grid = (unsigned)(a.static_ranks * batch * q_heads) + (unsigned)((a.dyn_items * 5 + 3) / 4);
  }
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (opt.exact && !opt.tail) attn256_kernel<true, false, false><<<grid, kA2Threads, 0, st>>>(a);
  else if (opt.exact) attn256_kernel<true, true, false><<<grid, kA2Threads, 0, st>>>(a);
  else attn256_kernel<false, true, true><<<grid, kA2Threads, 0, st>>>(a);
  return launch_status("attention_d256");
}

}  // namespace spx
