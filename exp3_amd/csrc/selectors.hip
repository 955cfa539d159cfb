// Balanced / CGF / dispersion block scores (kernels.py:49-126).
//
// For each real row r of tile t, head h and visible block j < t:
//   l0 = scale * q.mu_K,j + ln n_j
//   u  = max(0, scale^2 * (q*q).var_K,j)
//   logit = l0 (mean_balanced) | l0 + u / 2 (cgf_mean, dispersion_mean)
//   p = softmax over j < t ; contribution = p | p * sqrt(u) * sigma_V,j (dispersion)
//   score[t, j] = mean over the tile's real rows (0 for j >= t and for t = 0).
//
// gfx950 mapping
//   * The two dot products are MFMA GEMMs against the fp32 descriptors, kept to
//     about fp32 accuracy by splitting every fp32 operand into bf16 hi + lo parts
//     (q is bf16-exact; q*q is exact in fp32 and splits exactly into two bf16):
//       q.mu   = q.mu_hi + q.mu_lo                          (2 MFMA)
//       q2.var = q2_hi.var_hi + q2_hi.var_lo + q2_lo.var_hi (3 MFMA, drops 2^-16 term)
//   * selector_split_kernel splits mu_K and var_K once per call into a workspace
//     whose 32-block chunks are the LDS image the score kernel wants: per chunk and
//     128-dim half (one half at D = 128, two at D = 256), parts [mu hi, mu lo,
//     var hi, var lo] x 32 block rows x 128 dims bf16, 16-byte chunk c of row r at
//     position c ^ (r & 15) (bank-conflict-free operand reads).
//   * Scores are formed transposed (block j = MFMA row, query = lane column), so
//     the per-row softmax over blocks is an in-lane online reduction plus one
//     lane-half exchange, and the sum over the tile's rows is a transpose-reduction
//     across lanes (permlane / DPP, no LDS) plus a fixed-order add of the four row
//     groups' partial sums: the scores are the same on every call.
//   * Single pass: an item (tile, batch, q head) forms each chunk's products once.
//     Its logits stay in registers until the rows' softmax maximum and sum are
//     known; then exp2(logit - m) / l is summed per block. (dispersion_mean keeps
//     logit + log2(sqrt(u) sigma_V,j) instead, so the same exponent gives
//     p sqrt(u) sigma_V.) Rows with more chunks than the registers hold form the
//     products of the rest a second time.
//   * Persistent grid, one workgroup per CU, items heaviest first dealt round
//     robin. Descriptor chunks stream through two LDS buffers by direct
//     global->LDS loads (chunk s + 1 lands while chunk s is computed); the next
//     item's Q tile (into LDS, 16-byte chunk c of row r at c ^ (r & 15)) and first
//     chunk are copied while the current item finishes.
//   * selector_duo_kernel (mean_balanced, head_dim 128, up to 256 blocks): eight
//     waves, two per SIMD, two adjacent tiles of one head per item (waves 0-3 tile
//     t, waves 4-7 tile t - 1), each wave with all dims of its rows: every chunk
//     copy serves both tiles and no partial products are exchanged.
//   * selector_pair_kernel (cgf_mean and dispersion_mean, head_dim 128, up to 256
//     blocks; their q*q split leaves the duo kernel too few registers): eight
//     waves, two per SIMD. Waves w and w + 4 hold the same 32 query rows and split the 128 dims;
//     chunk jc belongs to the wave of the K half jc & 1, which adds its partner's
//     partial products (through one LDS slot per pair) to its own, folds the chunk
//     into its rows' softmax state beside the next chunk's products, and keeps the
//     chunk's logits.
//   * selector_kernel (head_dim 256, and longer rows): four waves, one per SIMD,
//     each with all dims of its 32 rows; the logits of the first S chunks are kept
//     in AGPRs (the MFMAs accumulate in VGPRs), a chunk's fold runs beside the next
//     chunk's products.
#include <algorithm>
#include <mutex>

#include "common.h"

namespace spx {

constexpr int kSelThreads = 256;
constexpr int kSelMaxBlocks = 1024;
constexpr int kSelChunk = 32;                          // blocks per chunk
constexpr int kSelPart = kSelChunk * 128;             // bf16 elements of one part (128-dim half)
constexpr int kSelChunkElems = 4 * kSelPart;           // 32 KB per 128-dim half of a chunk

struct SplitArgs {
  const float* mean_k;  // [B, NB, Hkv, D]
  const float* var_k;
  uint16_t* ws;         // [B, Hkv, NC, D / 128, 4, 32, 128] bf16
  int batch, kv_heads, blocks, chunks, dim;
  bool second_order;
  float mu_mul, var_mul;  // fp32 factors applied before the split (1 keeps the values)
};

__device__ __forceinline__ void split8(const float* v, u32x4& hi, u32x4& lo) {
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    const uint32_t h2 = pack_bf16x2(v[2 * e], v[2 * e + 1]);
    hi[e] = h2;
    lo[e] = pack_bf16x2(v[2 * e] - bf16_lo(h2), v[2 * e + 1] - bf16_hi(h2));
  }
}

// One thread per (b, g, block j of the padded range, 8-dim chunk c).
__global__ __launch_bounds__(256) void selector_split_kernel(SplitArgs a) {
  const int64_t id = (int64_t)blockIdx.x * 256 + threadIdx.x;
  const int cpr = a.dim / 8;   // 8-dim chunks per row
  const int64_t total = (int64_t)a.batch * a.kv_heads * a.chunks * kSelChunk * cpr;
  if (id >= total) return;
  const int c = (int)(id % cpr);
  const int64_t rest = id / cpr;
  const int jp = (int)(rest % ((int64_t)a.chunks * kSelChunk));
  const int64_t bg = rest / ((int64_t)a.chunks * kSelChunk);
  const int g = (int)(bg % a.kv_heads), b = (int)(bg / a.kv_heads);
  const int row = jp % kSelChunk, jc = jp / kSelChunk;
  float mu[8] = {}, var[8] = {};
  if (jp < a.blocks) {
    const int64_t off = (((int64_t)b * a.blocks + jp) * a.kv_heads + g) * a.dim + c * 8;
    const f32x4 m0 = *reinterpret_cast<const f32x4*>(a.mean_k + off);
    const f32x4 m1 = *reinterpret_cast<const f32x4*>(a.mean_k + off + 4);
#pragma unroll
    for (int x = 0; x < 4; ++x) { mu[x] = m0[x] * a.mu_mul; mu[4 + x] = m1[x] * a.mu_mul; }
    if (a.second_order) {
      const f32x4 v0 = *reinterpret_cast<const f32x4*>(a.var_k + off);
      const f32x4 v1 = *reinterpret_cast<const f32x4*>(a.var_k + off + 4);
#pragma unroll
      for (int x = 0; x < 4; ++x) { var[x] = v0[x] * a.var_mul; var[4 + x] = v1[x] * a.var_mul; }
    }
  }
  const int halves = a.dim / 128, hf = c >> 4, c16 = c & 15;
  uint16_t* dst = a.ws + (((bg * a.chunks + jc) * halves + hf) * kSelChunkElems) + row * 128 +
                  ((c16 ^ (row & 15)) << 3);
  u32x4 hi, lo;
  split8(mu, hi, lo);
  *reinterpret_cast<u32x4*>(dst) = hi;
  *reinterpret_cast<u32x4*>(dst + kSelPart) = lo;
  split8(var, hi, lo);
  *reinterpret_cast<u32x4*>(dst + 2 * kSelPart) = hi;
  *reinterpret_cast<u32x4*>(dst + 3 * kSelPart) = lo;
}

struct SelArgs {
  const uint16_t* q;
  int64_t qs_b, qs_s, qs_h;
  const uint16_t* ws;    // split descriptors, selector_split_kernel layout
  const float* sigma_v;  // [B, NB, Hkv]
  const int32_t* counts; // [NB]
  int batch, seq, q_heads, kv_heads, blocks, chunks;
  float scale;
  float* score;
  int64_t ss_b, ss_t, ss_j, ss_h;
};

template <int CTRL>
__device__ __forceinline__ float dpp(float x) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), CTRL, 0xf, 0xf, false));
}

// Sum 16 per-lane registers over the 32 lanes of each lane half; afterwards lane
// col (even) holds the sum of register 8 b4 + 4 b3 + 2 b2 + b1 (bits of col).
// Each step halves the registers a lane keeps: it keeps the half that its bit
// selects and adds the partner lane's copy of that half, the partner (opposite
// bit, same higher bits) sending the other half. Partners: lane ^ 16 through
// v_permlane16_swap (odd 16-lane rows of the first operand swapped with even rows
// of the second), then ^ 15, ^ 7, ^ 2, ^ 1 through DPP row mirror, half-row mirror
// and quad permutes; all vector ALU, no LDS round trips.
__device__ __forceinline__ float transpose_reduce16(float (&v)[16], int col) {
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const auto sw = __builtin_amdgcn_permlane16_swap(__float_as_uint(v[i]), __float_as_uint(v[i + 8]),
                                                     false, false);
    v[i] = __uint_as_float(sw[0]) + __uint_as_float(sw[1]);
  }
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const bool up = col & 8;
    const float keep = up ? v[i + 4] : v[i];
    const float send = up ? v[i] : v[i + 4];
    v[i] = keep + dpp<0x140>(send);   // row_mirror: lane ^ 15
  }
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    const bool up = col & 4;
    const float keep = up ? v[i + 2] : v[i];
    const float send = up ? v[i] : v[i + 2];
    v[i] = keep + dpp<0x141>(send);   // row_half_mirror: lane ^ 7
  }
  {
    const bool up = col & 2;
    const float keep = up ? v[1] : v[0];
    const float send = up ? v[0] : v[1];
    v[0] = keep + dpp<0x4e>(send);    // quad_perm [2, 3, 0, 1]: lane ^ 2
  }
  return v[0] + dpp<0xb1>(v[0]);      // quad_perm [1, 0, 3, 2]: lane ^ 1
}

// Copy NPART parts (NPART * 8 KB) of one workspace chunk into an LDS buffer with
// direct global->LDS loads: every lane moves 16 bytes per instruction, so one
// instruction of an NT-thread workgroup moves NT * 16 bytes. The consumer waits (vmcnt(0) and a
// barrier) before reading.
template <int NPART, int NT = kSelThreads>
__device__ __forceinline__ void dma_chunk(const uint16_t* src, uint16_t* lds, int tid) {
  const int w = tid >> 6;
  const uint32_t lds_base =
      (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) uint16_t*)lds;
  const uint32_t voff = (uint32_t)tid * 16u;
#pragma unroll
  for (int i = 0; i < NPART * 512 / NT; ++i) {
    const uint32_t m0 =
        __builtin_amdgcn_readfirstlane(lds_base + (uint32_t)(i * NT + w * 64) * 16u);
    const uint16_t* s = src + i * NT * 8;
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

// mu and var products of one 128-dim half (Q dims 128 HF ..) against the chunk
// image in LDS, accumulated into dmu / dvar. At D = 128 the q*q split comes from
// registers; at D = 256 it is formed from Q here (q*q is exact in fp32). The
// operand reads of k-step dc + 1 are issued before the products of dc (the
// scheduling groups keep them there), so each product finds its operand in
// registers instead of waiting out the LDS latency. between(dc) runs after the
// products of k-step dc: vector work that the groups spread between the products.
template <bool kSecond, int D, int HF, class Between>
__device__ __forceinline__ void selector_products(const uint16_t* ops, int e0,
                                                  const bf16x8 (&qb)[D / 16],
                                                  const bf16x8 (&q2h)[8], const bf16x8 (&q2l)[8],
                                                  f32x16& dmu, f32x16& dvar, Between&& between) {
  constexpr int kReads = kSecond ? 4 : 2;   // parts: mu hi, mu lo (, var hi, var lo)
  constexpr int kMfma = kSecond ? 5 : 2;
  u32x4 op[2][kReads];
  auto load = [&](int dc, u32x4 (&o)[kReads]) {
    const int off = e0 ^ (dc << 4);
#pragma unroll
    for (int p = 0; p < kReads; ++p) o[p] = *reinterpret_cast<const u32x4*>(ops + p * kSelPart + off);
  };
  load(0, op[0]);
  __builtin_amdgcn_sched_group_barrier(0x100, kReads, 0);   // DS reads
#pragma unroll
  for (int dc = 0; dc < 8; ++dc) {
    if (dc + 1 < 8) load(dc + 1, op[(dc + 1) & 1]);
    const u32x4(&o)[kReads] = op[dc & 1];
    const bf16x8 q = qb[HF * 8 + dc];
    dmu = mfma32(as_bf16x8(o[0]), q, dmu);
    dmu = mfma32(as_bf16x8(o[1]), q, dmu);
    if constexpr (kSecond) {
      bf16x8 sh, sl;
      if (D == 128) {
        sh = q2h[dc];
        sl = q2l[dc];
      } else {
        // opaque copy: the split is formed here for every use instead of being
        // hoisted out of the chunk loop (which would hold 128 more registers)
        u32x4 raw = __builtin_bit_cast(u32x4, q);
        asm volatile("" : "+v"(raw));
        float sq[8];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const float x0 = bf16_lo(raw[e]), x1 = bf16_hi(raw[e]);
          sq[2 * e] = x0 * x0;
          sq[2 * e + 1] = x1 * x1;
        }
        u32x4 hi, lo;
        split8(sq, hi, lo);
        sh = as_bf16x8(hi);
        sl = as_bf16x8(lo);
      }
      const bf16x8 vh = as_bf16x8(o[2]), vl = as_bf16x8(o[3]);
      dvar = mfma32(vh, sh, dvar);
      dvar = mfma32(vl, sh, dvar);
      dvar = mfma32(vh, sl, dvar);
    }
    between(dc);
    if (dc + 1 < 8) __builtin_amdgcn_sched_group_barrier(0x100, kReads, 0);
    // each product followed by a few vector instructions
#pragma unroll
    for (int m = 0; m < kMfma; ++m) {
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);    // MFMA
      __builtin_amdgcn_sched_group_barrier(0x402, 4, 0);    // VALU incl. exp
    }
  }
}

// Per-lane gather into LDS: 16 bytes from this lane's own address land at
// lds_wave + 16 x lane (lds_wave uniform over the wave); awaited with vmcnt.
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

// The 128 x D query tile of (b, t, h) into LDS, 16-byte chunk c of row r at
// position c ^ (r & 15) of its row (conflict-free operand reads). Rows past the
// sequence end are clamped to the last row (the readers zero them).
template <int D, int NT = kSelThreads>
__device__ __forceinline__ void dma_q(const SelArgs& a, int t, int b, int h, uint16_t* qbuf,
                                      int tid) {
  constexpr int kRowChunks = D / 8;
  constexpr int kInsts = kBlock * kRowChunks / NT;
  const int w = tid >> 6;
  const uint32_t lds_base =
      (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) uint16_t*)qbuf;
  const uint16_t* base = a.q + (int64_t)b * a.qs_b + (int64_t)h * a.qs_h;
  const int last = a.seq - 1;
#pragma unroll
  for (int i = 0; i < kInsts; ++i) {
    const int p = i * NT + tid;
    const int r = p / kRowChunks, c = (p % kRowChunks) ^ (r & 15);
    const int64_t row = min(t * kBlock + r, last);
    dma_gather16(base + row * a.qs_s + c * 8, lds_base + (uint32_t)(i * NT + w * 64) * 16u);
  }
}

// This lane's Q operand registers (row 32 w + col, 16-byte chunks 2 dc + half) from
// the LDS tile, zero past the sequence end; at D = 128 also the exact bf16 hi/lo
// split of q * q.
template <bool kSecond, int D>
__device__ __forceinline__ void read_q(const uint16_t* qbuf, int w, int col, int half, bool row_ok,
                                       bf16x8 (&qb)[D / 16], bf16x8 (&q2h)[8], bf16x8 (&q2l)[8]) {
  const int r = w * 32 + col;
#pragma unroll
  for (int dc = 0; dc < D / 16; ++dc) {
    const int c = 2 * dc + half;
    u32x4 raw = *reinterpret_cast<const u32x4*>(qbuf + r * D + ((c ^ (r & 15)) << 3));
    if (!row_ok) raw = u32x4{0u, 0u, 0u, 0u};
    qb[dc] = as_bf16x8(raw);
    if (kSecond && D == 128) {
      float sq[8];
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const float x0 = bf16_lo(raw[e]), x1 = bf16_hi(raw[e]);
        sq[2 * e] = x0 * x0;
        sq[2 * e + 1] = x1 * x1;
      }
      u32x4 hi, lo;
      split8(sq, hi, lo);
      q2h[dc & 7] = as_bf16x8(hi);
      q2l[dc & 7] = as_bf16x8(lo);
    }
  }
}

// Persistent item deal. Items are (rank, bh): rank 0 the heaviest tile (or tile
// pair), bh = batch * Hq + head. Workgroup w runs on XCD w % 8 (the hardware deals
// workgroup ids round robin over the 8 XCDs; the grid is a multiple of 8); the
// workgroups of XCD x take the ranks x, x + 8, x + 16, ... with all their heads, in
// turn. All heads of a rank thus run on one XCD, so the partial cache lines of the
// head-interleaved score rows ([B, NB, NB, Hq], 4 bytes per head) meet in one L2
// instead of leaving it as 32-byte partial writes from every XCD. Returns the m-th
// item of workgroup w (an index >= ranks * per_rank once the ranks are used up).
__device__ __forceinline__ int xcd_item(int w, int m, int nwg, int per_rank) {
  const int x = w & 7, k = w >> 3, per_xcd = nwg >> 3;
  const int idx = k + m * per_xcd;
  return (x + 8 * (idx / per_rank)) * per_rank + idx % per_rank;
}

// The deal of the long-row kernel when the B * Hkv (batch, kv group) streams divide
// the 8 XCDs: stream s runs on XCDs s X .. s X + X - 1 (X = 8 / streams), which
// take its ranks in turn (rank u, u + X, ... on the stream's u-th XCD) with the
// group's heads. An XCD then holds one stream's descriptor chunks in its L2
// (1 MB per stream at 131072 tokens) instead of every stream's. Returns the item
// (rank * per_rank + b * Hq + head) or an index >= ranks * per_rank when done.
__device__ __forceinline__ int xcd_item_stream(int w, int m, int nwg, int streams, int group,
                                               int kv_heads, int q_heads, int ranks) {
  const int x = w & 7, k = w >> 3, per_xcd = nwg >> 3;
  const int X = 8 / streams, st = x / X, u = x % X;
  const int idx = k + m * per_xcd;
  const int rank = u + X * (idx / group);
  if (rank >= ranks) return ranks * q_heads * (streams / kv_heads);
  const int b = st / kv_heads, g = st % kv_heads;
  return rank * (q_heads * (streams / kv_heads)) + b * q_heads + g * group + idx % group;
}

// A value parked in an accumulation register (AGPR) until the end of the item:
// the kernel's MFMAs use VGPR accumulators, so the AGPR file holds the logits of
// the stored chunks.
__device__ __forceinline__ float park(float v) {
  float r;
  asm("v_accvgpr_write_b32 %0, %1" : "=a"(r) : "v"(v));
  return r;
}

__device__ __forceinline__ float unpark(float a) {
  float r;
  asm("v_accvgpr_read_b32 %0, %1" : "=v"(r) : "a"(a));
  return r;
}

struct SelConsts {
  float scale_l2, scale2_half_l2, scale2;
};

// Logits of chunk jc in log2 units, (scale q.mu + ln n + u / 2) * log2 e, with
// the blocks j >= t masked to -inf (only in the last chunk). `val` is what the end
// phase exponentiates: the logit itself, or for dispersion_mean the logit plus
// log2(sqrt(u) sigma_V,j), so that exp2(val - m) / l = p * sqrt(u) * sigma_V,j.
// Rows past the sequence end (Q = 0) give finite logits and are dropped later.
template <bool kSecond, bool kDisp>
__device__ __forceinline__ void chunk_logits(const f32x16& dmu, const f32x16& dvar, int jc, int t,
                                             int lane, const float* log2_n,
                                             const float* log2_sigma, const SelConsts& k,
                                             float (&lg)[16], float (&val)[16]) {
  const int lim = t - jc * kSelChunk;  // visible rows of this chunk: jr < lim
#pragma unroll
  for (int r = 0; r < 16; ++r) {
    const int jr = mfma32_row(r, lane);
    const int j = jc * kSelChunk + jr;
    float l2 = fmaf(dmu[r], k.scale_l2, log2_n[j]);
    const float u = fmaxf(dvar[r], 0.0f);
    if (kSecond) l2 = fmaf(u, k.scale2_half_l2, l2);
    const bool vis = jr < lim;
    lg[r] = vis ? l2 : -INFINITY;
    if (kDisp) val[r] = vis ? l2 + 0.5f * __log2f(u * k.scale2) + log2_sigma[j] : -INFINITY;
  }
}

// Fold 16 logits of this lane's row into its online softmax state (log2 units).
// Branch-free (selects in place of a test on the new maximum); a row with no
// finite logit yet keeps m = -inf and l = 0.
__device__ __forceinline__ void fold_row(const float (&lg)[16], float& m_run, float& l_run) {
  float mx = -INFINITY;
#pragma unroll
  for (int r = 0; r < 16; ++r) mx = fmaxf(mx, lg[r]);
  const float m_new = fmaxf(m_run, mx);
  const float base = m_new == -INFINITY ? 0.0f : m_new;
  float sum = 0.0f;
#pragma unroll
  for (int r = 0; r < 16; ++r) sum += exp2_fast(lg[r] - base);
  const float keep = m_run == -INFINITY ? 0.0f : exp2_fast(m_run - base);
  l_run = l_run * keep + sum;
  m_run = m_new;
}

// chunk_logits + fold_row + parking of one stored chunk whose blocks are all
// visible (no mask needed), cut into eight pieces
// that run between the next chunk's k-steps (piece(dc) after k-step dc): pieces
// 0-3 form four logits each and their maximum, pieces 4-7 exponentiate and park
// four each; the same operations in the same order as the unpieced functions.
template <bool kSecond, bool kDisp>
struct ChunkFold {   // for chunks with all 32 blocks visible (j < t)
  const f32x16& dmu;
  const f32x16& dvar;
  int jc, lane;
  const float* log2_n;
  const float* log2_sigma;
  const SelConsts& k;
  float lg[16], val[16];
  float mx = -INFINITY, m_new = 0.0f, base = 0.0f, keep = 0.0f, sum = 0.0f;

  __device__ __forceinline__ void piece(int dc, float& m_run, float& l_run, float (&st)[16]) {
    if (dc < 4) {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int r = 4 * dc + i;
        const int j = jc * kSelChunk + mfma32_row(r, lane);
        float l2 = fmaf(dmu[r], k.scale_l2, log2_n[j]);
        const float u = fmaxf(dvar[r], 0.0f);
        if (kSecond) l2 = fmaf(u, k.scale2_half_l2, l2);
        lg[r] = l2;
        if (kDisp) val[r] = l2 + 0.5f * __log2f(u * k.scale2) + log2_sigma[j];
        mx = fmaxf(mx, lg[r]);
      }
    } else {
      if (dc == 4) {
        m_new = fmaxf(m_run, mx);
        base = m_new == -INFINITY ? 0.0f : m_new;
        keep = m_run == -INFINITY ? 0.0f : exp2_fast(m_run - base);
      }
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int r = 4 * (dc - 4) + i;
        sum += exp2_fast(lg[r] - base);
        st[r] = park(kDisp ? val[r] : lg[r]);
      }
      if (dc == 7) {
        l_run = l_run * keep + sum;
        m_run = m_new;
      }
    }
  }
};

// Normalised contributions of one chunk, summed over the wave's 32 query rows per
// block into part[w][block].
template <int NBMAX>
__device__ __forceinline__ void chunk_sums(float (&v)[16], float m, float inv_l, int jc, int w,
                                           int lane, float (*part)[NBMAX]) {
  const int col = lane & 31;
#pragma unroll
  for (int r = 0; r < 16; ++r) v[r] = exp2_fast(v[r] - m) * inv_l;
  const float total = transpose_reduce16(v, col);
  if ((col & 1) == 0) {
    const int R = 8 * ((col >> 4) & 1) + 4 * ((col >> 3) & 1) + 2 * ((col >> 2) & 1) + ((col >> 1) & 1);
    part[w][jc * kSelChunk + mfma32_row(R, lane)] = total;
  }
}

// One persistent workgroup per CU, four waves (one per SIMD) of 32 query rows;
// items (query tile t, batch b, q head h) heaviest first, dealt round robin. Each
// item is a single pass over its visible block chunks: the logits of the first S
// chunks stay in AGPRs (16 per lane and chunk) until the row's softmax maximum and
// sum are known, and only chunks past S (more than 32 S visible blocks) have their
// products formed a second time. The descriptor chunks stream through two LDS
// buffers; the next item's Q tile and first chunk are copied in while the current
// item's last step and its sums run. A chunk's softmax fold runs beside the next
// chunk's products.
template <int SEL, int D, int S>
__global__ __launch_bounds__(kSelThreads, 1) void selector_kernel(SelArgs args) {
  constexpr bool kSecond = SEL != SPX_SELECTOR_MEAN_BALANCED;
  constexpr bool kDisp = SEL == SPX_SELECTOR_DISPERSION_MEAN;
  constexpr int kParts = kSecond ? 4 : 2;
  constexpr int kHalves = D / 128;

  __shared__ __align__(16) uint16_t buf[2][kParts * kSelPart];
  __shared__ __align__(16) uint16_t qbuf[kBlock * D];
  __shared__ float log2_n[kSelMaxBlocks];
  __shared__ float log2_sigma[kDisp ? kSelMaxBlocks : 1];
  __shared__ float part[4][kSelMaxBlocks];

  {
    const int tid = threadIdx.x;
    for (int j = tid; j < args.blocks; j += kSelThreads) log2_n[j] = log2f((float)args.counts[j]);
    const int per_tile = args.batch * args.q_heads;
    const int streams = args.batch * args.kv_heads;
    const int item = 8 % streams == 0
        ? xcd_item_stream(blockIdx.x, 0, gridDim.x, streams, args.q_heads / args.kv_heads,
                          args.kv_heads, args.q_heads, args.blocks)
        : xcd_item(blockIdx.x, 0, gridDim.x, per_tile);
    if (item < args.blocks * per_tile) {
      const int t = args.blocks - 1 - item / per_tile, bh = item % per_tile;
      const int b = bh / args.q_heads, h = bh % args.q_heads;
      dma_q<D>(args, t, b, h, qbuf, tid);
      if (t > 0) {
        const int64_t bg_elems = (int64_t)args.chunks * kHalves * kSelChunkElems;
        dma_chunk<kParts>(args.ws + ((int64_t)b * args.kv_heads + h / (args.q_heads / args.kv_heads)) * bg_elems,
                          buf[0], tid);
      }
    }
  }
  int slot = 0;  // buffer of the current item's first step

  for (int m = 0;; ++m) {
    // The arguments are read afresh for every item through an opaque pointer and the
    // thread index through an opaque copy, so nothing derived from them is held in
    // registers across items.
#if defined(__HIP_DEVICE_COMPILE__)
    const __attribute__((address_space(4))) SelArgs* ap =
        (const __attribute__((address_space(4))) SelArgs*)__builtin_amdgcn_kernarg_segment_ptr();
    asm volatile("" : "+s"(ap));
    const SelArgs a = *ap;
#else
    const SelArgs a = args;
#endif
    const int per_tile = a.batch * a.q_heads;
    const int n_items = a.blocks * per_tile;
    const int streams = a.batch * a.kv_heads;
    const bool by_stream = 8 % streams == 0;
    auto deal = [&](int mm) {
      return by_stream ? xcd_item_stream(blockIdx.x, mm, gridDim.x, streams,
                                         a.q_heads / a.kv_heads, a.kv_heads, a.q_heads, a.blocks)
                       : xcd_item(blockIdx.x, mm, gridDim.x, per_tile);
    };
    const int item = deal(m);
    if (item >= n_items) break;
    const int tid = opaque((int)threadIdx.x), lane = tid & 63, w = tid >> 6;
    const int col = lane & 31, half = lane >> 5;
    const int group = a.q_heads / a.kv_heads;
    const int64_t bg_elems = (int64_t)a.chunks * kHalves * kSelChunkElems;
    const SelConsts k{a.scale * kLog2e, 0.5f * a.scale * a.scale * kLog2e, a.scale * a.scale};
    // LDS element offset of this lane's operand row (block col) at 16-byte chunk
    // 2 dc + half: (2 dc + half) ^ (col & 15) = base ^ (dc << 4) in elements.
    const int e0 = col * 128 + (((col >> 1) & 7) << 4) + ((half ^ (col & 1)) << 3);

    const int t = a.blocks - 1 - item / per_tile, bh = item % per_tile;
    const int b = bh / a.q_heads, h = bh % a.q_heads, g = h / group;
    const int nchunks = (t + kSelChunk - 1) / kSelChunk;  // visible blocks j < t
    const int nstored = min(nchunks, S);
    const int p1 = nchunks * kHalves;                     // first-pass (chunk, half) steps
    const int nsteps = p1 + (nchunks - nstored) * kHalves;
    const uint16_t* src = a.ws + ((int64_t)b * a.kv_heads + g) * bg_elems;
    const int next = deal(m + 1);

    // Copy what step s + 1 reads into its buffer: this item's next (chunk, half),
    // or after the last step the next item's Q tile and first step. Called after
    // the barrier that opens step s, when every wave is done with step s - 1.
    auto issue_after = [&](int s) {
      uint16_t* dst = buf[(slot + s + 1) & 1];
      if (s + 1 < nsteps) {
        const int s1 = s + 1;
        const int jc = s1 < p1 ? s1 / kHalves : nstored + (s1 - p1) / kHalves;
        dma_chunk<kParts>(src + (int64_t)(jc * kHalves + s1 % kHalves) * kSelChunkElems, dst, tid);
      } else if (next < n_items) {
        const int nt = a.blocks - 1 - next / per_tile, nbh = next % per_tile;
        const int nb = nbh / a.q_heads, nh = nbh % a.q_heads;
        dma_q<D>(a, nt, nb, nh, qbuf, tid);
        if (nt > 0) dma_chunk<kParts>(a.ws + ((int64_t)nb * a.kv_heads + nh / group) * bg_elems, dst, tid);
      }
    };
    auto step_sync = [&]() {
      asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
      block_sync();
    };

    step_sync();  // Q and the first step landed; the previous item's LDS reads are done
    const int64_t qrow = (int64_t)t * kBlock + w * 32 + col;
    const bool row_ok = qrow < a.seq;
    bf16x8 qb[D / 16], q2h[8], q2l[8];
    read_q<kSecond, D>(qbuf, w, col, half, row_ok, qb, q2h, q2l);
    if (kDisp) {
      for (int j = tid; j < t; j += kSelThreads)
        log2_sigma[j] = __log2f(a.sigma_v[((int64_t)b * a.blocks + j) * a.kv_heads + g]);
    }
    block_sync();  // the Q tile is free for the next item's copy; log2_sigma visible
    if (nsteps == 0) issue_after(-1);

    float m_run = -INFINITY, l_run = 0.0f;  // this lane's row state over its blocks
    float st[S][16];                         // parked logits of the stored chunks
    f32x16 acc_mu[2], acc_var[2];            // products of chunk jc in set jc & 1

    // ---- stored chunks: products, the previous chunk's fold beside them
#pragma unroll
    for (int jc = 0; jc < S; ++jc) {
      if (jc < nstored) {
        f32x16& dmu = acc_mu[jc & 1];
        f32x16& dvar = acc_var[jc & 1];
#pragma unroll
        for (int hf = 0; hf < kHalves; ++hf) {
          const int sc = jc * kHalves + hf;
          if (sc > 0) step_sync();
          issue_after(sc);
          const uint16_t* ops = buf[(slot + sc) & 1];
          if (hf == 0) {
            dmu = f32x16{};
            dvar = f32x16{};
            if (jc > 0) {
              // the previous chunk's fold, in pieces between this chunk's products
              ChunkFold<kSecond, kDisp> f{acc_mu[(jc - 1) & 1], acc_var[(jc - 1) & 1], jc - 1,
                                          lane, log2_n, log2_sigma, k};
              selector_products<kSecond, D, 0>(ops, e0, qb, q2h, q2l, dmu, dvar, [&](int dc) {
                f.piece(dc, m_run, l_run, st[jc - 1]);
              });
            } else {
              selector_products<kSecond, D, 0>(ops, e0, qb, q2h, q2l, dmu, dvar, [](int) {});
            }
          } else {
            selector_products<kSecond, D, kHalves - 1>(ops, e0, qb, q2h, q2l, dmu, dvar,
                                                       [](int) {});
          }
        }
        if (jc + 1 == nstored) {
          float lg[16], val[16];
          chunk_logits<kSecond, kDisp>(dmu, dvar, jc, t, lane, log2_n, log2_sigma, k, lg, val);
          fold_row(lg, m_run, l_run);
#pragma unroll
          for (int r = 0; r < 16; ++r) st[jc][r] = park(kDisp ? val[r] : lg[r]);
        }
      }
    }
    // ---- chunks past S, first pass: the row state only
    for (int jc = S; jc < nchunks; ++jc) {
      f32x16 dmu = {}, dvar = {};
      for (int hf = 0; hf < kHalves; ++hf) {
        const int sc = jc * kHalves + hf;
        step_sync();
        issue_after(sc);
        const uint16_t* ops = buf[(slot + sc) & 1];
        if (hf == 0) selector_products<kSecond, D, 0>(ops, e0, qb, q2h, q2l, dmu, dvar, [](int) {});
        else selector_products<kSecond, D, kHalves - 1>(ops, e0, qb, q2h, q2l, dmu, dvar, [](int) {});
      }
      float lg[16], val[16];
      chunk_logits<kSecond, kDisp>(dmu, dvar, jc, t, lane, log2_n, log2_sigma, k, lg, val);
      fold_row(lg, m_run, l_run);
    }

    // ---- the row's softmax maximum and sum: merge the two lane halves
    float inv_l;
    {
      const float om = xor32(m_run), ol = xor32(l_run);
      const float nm = fmaxf(m_run, om);
      float nl = 0.0f;
      if (nm != -INFINITY) {
        nl = (m_run == -INFINITY ? 0.0f : l_run * exp2_fast(m_run - nm)) +
             (om == -INFINITY ? 0.0f : ol * exp2_fast(om - nm));
      }
      m_run = nm;
      // rows past the sequence end contribute nothing
      inv_l = (nl > 0.0f && row_ok) ? 1.0f / nl : 0.0f;
    }
#pragma unroll
    for (int jc = 0; jc < S; ++jc) {
      if (jc < nstored) {
        float v[16];
#pragma unroll
        for (int r = 0; r < 16; ++r) v[r] = unpark(st[jc][r]);
        chunk_sums(v, m_run, inv_l, jc, w, lane, part);
      }
    }
    // ---- chunks past S, second pass: products again, then their sums
    for (int jc = nstored; jc < nchunks; ++jc) {
      f32x16 dmu = {}, dvar = {};
      for (int hf = 0; hf < kHalves; ++hf) {
        const int sc = p1 + (jc - nstored) * kHalves + hf;
        step_sync();
        issue_after(sc);
        const uint16_t* ops = buf[(slot + sc) & 1];
        if (hf == 0) selector_products<kSecond, D, 0>(ops, e0, qb, q2h, q2l, dmu, dvar, [](int) {});
        else selector_products<kSecond, D, kHalves - 1>(ops, e0, qb, q2h, q2l, dmu, dvar, [](int) {});
      }
      float lg[16], val[16];
      chunk_logits<kSecond, kDisp>(dmu, dvar, jc, t, lane, log2_n, log2_sigma, k, lg, val);
      if constexpr (kDisp) chunk_sums(val, m_run, inv_l, jc, w, lane, part);
      else chunk_sums(lg, m_run, inv_l, jc, w, lane, part);
    }

    block_sync();  // every wave's block sums are in part
    const float inv_rows = 1.0f / (float)min(kBlock, a.seq - t * kBlock);
    for (int j = tid; j < a.blocks; j += kSelThreads) {
      const float sc = j < t ? (part[0][j] + part[1][j] + part[2][j] + part[3][j]) * inv_rows : 0.0f;
      a.score[b * a.ss_b + t * a.ss_t + j * a.ss_j + h * a.ss_h] = sc;
    }
    slot = (slot + nsteps) & 1;
  }
}

// ---------------------------------------------------------------------------
// head_dim 128: two waves per SIMD.
//
// One persistent workgroup of eight waves per CU. Waves w and w + 4 hold the same
// 32 query rows (row group w & 3) and split the 128 dims: wave w + 4 kh forms the
// products of dims 64 kh .. 64 kh + 63 (k-steps 4 kh .. 4 kh + 3). Chunk jc belongs
// to the wave with kh == jc & 1: the other wave leaves its partial products in the
// pair's LDS exchange slot, and the owner adds them to its own (the two partial
// sums meet in one fp32 addition, the same whichever wave owns the chunk), folds
// the chunk into its rows' softmax state and parks its logits. A chunk's owner is
// the non-owner of the next chunk, so within one step the same wave first reads the
// slot (the previous chunk's partner products, beside this chunk's products) and
// then writes it: one slot per pair, no second buffer. Two waves per SIMD let one
// wave's softmax and reduction instructions issue beside the other's products.

constexpr int kPairThreads = 512;

// The products of this wave's four k-steps (dims 64 kh ..) against the chunk
// image in LDS; e0k is the operand offset with kh folded in. between(dc) runs after
// k-step dc, its vector instructions spread between the products. (The second wave
// on the SIMD covers the operand reads' latency: a read-ahead register set cost
// more registers than the pair of waves can spare.)
template <bool kSecond, class Between>
__device__ __forceinline__ void pair_products(const uint16_t* ops, int e0k, const bf16x8 (&qb)[4],
                                              const bf16x8 (&q2h)[4], const bf16x8 (&q2l)[4],
                                              f32x16& dmu, f32x16& dvar, Between&& between) {
  constexpr int kMfma = kSecond ? 5 : 2;
#pragma unroll
  for (int dc = 0; dc < 4; ++dc) {
    const int off = e0k ^ (dc << 4);
    const bf16x8 mh = as_bf16x8(*reinterpret_cast<const u32x4*>(ops + off));
    const bf16x8 ml = as_bf16x8(*reinterpret_cast<const u32x4*>(ops + kSelPart + off));
    dmu = mfma32(mh, qb[dc], dmu);
    dmu = mfma32(ml, qb[dc], dmu);
    if constexpr (kSecond) {
      const bf16x8 vh = as_bf16x8(*reinterpret_cast<const u32x4*>(ops + 2 * kSelPart + off));
      const bf16x8 vl = as_bf16x8(*reinterpret_cast<const u32x4*>(ops + 3 * kSelPart + off));
      dvar = mfma32(vh, q2h[dc], dvar);
      dvar = mfma32(vl, q2h[dc], dvar);
      dvar = mfma32(vh, q2l[dc], dvar);
    }
    between(dc);
#pragma unroll
    for (int m = 0; m < kMfma; ++m) {
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
      __builtin_amdgcn_sched_group_barrier(0x402, 4, 0);
    }
  }
}

// A pair's exchange slot: 16-byte chunk i of lane l at xs + 4 (64 i + l) floats;
// chunks 0-3 hold dmu[4 i ..], chunks 4-7 dvar[4 (i - 4) ..].
template <bool kSecond>
__device__ __forceinline__ void put_partial(float* xs, int lane, const f32x16& dmu,
                                            const f32x16& dvar) {
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    *reinterpret_cast<f32x4*>(xs + (i * 64 + lane) * 4) =
        f32x4{dmu[4 * i], dmu[4 * i + 1], dmu[4 * i + 2], dmu[4 * i + 3]};
    if constexpr (kSecond)
      *reinterpret_cast<f32x4*>(xs + ((4 + i) * 64 + lane) * 4) =
          f32x4{dvar[4 * i], dvar[4 * i + 1], dvar[4 * i + 2], dvar[4 * i + 3]};
  }
}

// Add the partner's partial products of registers 4 i .. 4 i + 3.
template <bool kSecond>
__device__ __forceinline__ void add_partial(const float* xs, int lane, int i, f32x16& dmu,
                                            f32x16& dvar) {
  const f32x4 a = *reinterpret_cast<const f32x4*>(xs + (i * 64 + lane) * 4);
#pragma unroll
  for (int e = 0; e < 4; ++e) dmu[4 * i + e] += a[e];
  if constexpr (kSecond) {
    const f32x4 b = *reinterpret_cast<const f32x4*>(xs + ((4 + i) * 64 + lane) * 4);
#pragma unroll
    for (int e = 0; e < 4; ++e) dvar[4 * i + e] += b[e];
  }
}

// The owner's fold of a fully visible chunk, in four pieces run between the next
// chunk's k-steps: pieces 0-1 add the partner's products of eight registers each
// and form their logits (kept in st) and maximum, pieces 2-3 exponentiate eight
// each (the operations and order of chunk_logits + fold_row).
template <bool kSecond, bool kDisp>
struct PairFold {
  f32x16& dmu;
  f32x16& dvar;
  const float* xs;
  int jc, lane;
  const float* log2_n;
  const float* log2_sigma;
  const SelConsts& k;
  float lg[kDisp ? 16 : 1];   // dispersion: the logits (st holds the exponents)
  float mx = -INFINITY, m_new = 0.0f, base = 0.0f, keep = 0.0f, sum = 0.0f;

  __device__ __forceinline__ void piece(int p, float& m_run, float& l_run, float (&st)[16]) {
    if (p < 2) {
      add_partial<kSecond>(xs, lane, 2 * p, dmu, dvar);
      add_partial<kSecond>(xs, lane, 2 * p + 1, dmu, dvar);
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const int r = 8 * p + i;
        const int j = jc * kSelChunk + mfma32_row(r, lane);
        float l2 = fmaf(dmu[r], k.scale_l2, log2_n[j]);
        const float u = fmaxf(dvar[r], 0.0f);
        if (kSecond) l2 = fmaf(u, k.scale2_half_l2, l2);
        if constexpr (kDisp) {
          lg[r] = l2;
          st[r] = l2 + 0.5f * __log2f(u * k.scale2) + log2_sigma[j];
        } else {
          st[r] = l2;
        }
        mx = fmaxf(mx, l2);
      }
    } else {
      if (p == 2) {
        m_new = fmaxf(m_run, mx);
        base = m_new == -INFINITY ? 0.0f : m_new;
        keep = m_run == -INFINITY ? 0.0f : exp2_fast(m_run - base);
      }
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const int r = 8 * (p - 2) + i;
        sum += exp2_fast((kDisp ? lg[r] : st[r]) - base);
      }
      if (p == 3) {
        l_run = l_run * keep + sum;
        m_run = m_new;
      }
    }
  }
};

// The pair kernel's LDS.
struct PairLds {
  uint16_t (*buf)[4 * kSelPart];
  uint16_t* qbuf;
  float (*xbuf)[8 * 64 * 4];
  float* log2_n;
  float* log2_sigma;
  float (*part)[kSelMaxBlocks];
  float2 (*rowstate)[kBlock];
};

// The item loop of the waves with dims 64 KH .. 64 KH + 63. Both halves of the
// workgroup run it over the same items and meet at the same barriers; chunk jc is
// owned by the half with KH == jc & 1, so every ownership test is resolved at
// compile time.
template <int SEL, int S, int KH>
__device__ __forceinline__ void pair_waves(const SelArgs& args, const PairLds& L) {
  constexpr bool kSecond = SEL != SPX_SELECTOR_MEAN_BALANCED;
  constexpr bool kDisp = SEL == SPX_SELECTOR_DISPERSION_MEAN;
  constexpr int kParts = kSecond ? 4 : 2;
  int slot = 0;  // buffer of the current item's first step

  for (int m = 0;; ++m) {
    // arguments re-read per item through an opaque pointer, the thread index through
    // an opaque copy: nothing derived from them is held across items
#if defined(__HIP_DEVICE_COMPILE__)
    const __attribute__((address_space(4))) SelArgs* ap =
        (const __attribute__((address_space(4))) SelArgs*)__builtin_amdgcn_kernarg_segment_ptr();
    asm volatile("" : "+s"(ap));
    const SelArgs a = *ap;
#else
    const SelArgs a = args;
#endif
    const int per_tile = a.batch * a.q_heads;
    const int n_items = a.blocks * per_tile;
    const int item = xcd_item(blockIdx.x, m, gridDim.x, per_tile);
    if (item >= n_items) break;
    const int tid = opaque((int)threadIdx.x), lane = tid & 63;
    const int rg = (tid >> 6) & 3;  // row group
    const int col = lane & 31, half = lane >> 5;
    const int group = a.q_heads / a.kv_heads;
    const int64_t bg_elems = (int64_t)a.chunks * kSelChunkElems;
    const SelConsts k{a.scale * kLog2e, 0.5f * a.scale * a.scale * kLog2e, a.scale * a.scale};
    const int e0k = (col * 128 + (((col >> 1) & 7) << 4) + ((half ^ (col & 1)) << 3)) ^ (KH << 6);

    const int t = a.blocks - 1 - item / per_tile, bh = item % per_tile;
    const int b = bh / a.q_heads, h = bh % a.q_heads, g = h / group;
    const int nchunks = (t + kSelChunk - 1) / kSelChunk;  // visible blocks j < t
    const int nstored = min(nchunks, S);
    const int nsteps = nchunks + (nchunks - nstored);     // pass 1, then pass 2 past S
    const uint16_t* src = a.ws + ((int64_t)b * a.kv_heads + g) * bg_elems;
    const int next = xcd_item(blockIdx.x, m + 1, gridDim.x, per_tile);

    // Copy this item's step s + 1 into its buffer; called after the barrier that
    // opens step s, when every wave is done with step s - 1.
    auto issue_after = [&](int s) {
      if (s + 1 < nsteps) {
        const int s1 = s + 1;
        const int jc = s1 < nchunks ? s1 : nstored + (s1 - nchunks);
        dma_chunk<kParts, kPairThreads>(src + (int64_t)jc * kSelChunkElems,
                                        L.buf[(slot + s1) & 1], tid);
      }
    };
    // The next item's Q tile and first chunk, issued once this item's last step has
    // been opened (its buffer, the other one, and the Q tile are free by then).
    auto issue_next_item = [&]() {
      if (next < n_items) {
        const int nt = a.blocks - 1 - next / per_tile, nbh = next % per_tile;
        const int nb = nbh / a.q_heads, nh = nbh % a.q_heads;
        dma_q<128, kPairThreads>(a, nt, nb, nh, L.qbuf, tid);
        if (nt > 0)
          dma_chunk<kParts, kPairThreads>(a.ws + ((int64_t)nb * a.kv_heads + nh / group) * bg_elems,
                                          L.buf[(slot + nsteps) & 1], tid);
      }
    };
    auto step_sync = [&]() {
      asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
      block_sync();
    };

    step_sync();  // Q and the first chunk landed; the previous item's LDS reads are done
    const int64_t qrow = (int64_t)t * kBlock + rg * 32 + col;
    const bool row_ok = qrow < a.seq;
    bf16x8 qb[4], q2h[4], q2l[4];
    {
      const int r = rg * 32 + col;
#pragma unroll
      for (int dc = 0; dc < 4; ++dc) {
        const int c = 2 * (4 * KH + dc) + half;
        u32x4 raw = *reinterpret_cast<const u32x4*>(L.qbuf + r * 128 + ((c ^ (r & 15)) << 3));
        if (!row_ok) raw = u32x4{0u, 0u, 0u, 0u};
        qb[dc] = as_bf16x8(raw);
        if (kSecond) {
          float sq[8];
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            const float x0 = bf16_lo(raw[e]), x1 = bf16_hi(raw[e]);
            sq[2 * e] = x0 * x0;
            sq[2 * e + 1] = x1 * x1;
          }
          u32x4 hi, lo;
          split8(sq, hi, lo);
          q2h[dc] = as_bf16x8(hi);
          q2l[dc] = as_bf16x8(lo);
        }
      }
    }
    if (kDisp) {
      for (int j = tid; j < t; j += kPairThreads)
        L.log2_sigma[j] = __log2f(a.sigma_v[((int64_t)b * a.blocks + j) * a.kv_heads + g]);
    }
    block_sync();  // the Q tile is free for the next item's copy; log2_sigma visible
    if (nsteps == 0) issue_next_item();

    float* xs = L.xbuf[rg];
    float m_run = -INFINITY, l_run = 0.0f;   // this lane's row state over its own chunks
    float st[S / 2][16] = {};                // logits of this half's stored chunks
    f32x16 acc_mu[2] = {}, acc_var[2] = {};  // products of chunk jc in set jc & 1

    // ---- stored chunks
#pragma unroll
    for (int jc = 0; jc < S; ++jc) {
      if (jc < nstored) {
        const bool mine = KH == (jc & 1);  // compile time once unrolled
        f32x16& dmu = acc_mu[jc & 1];
        f32x16& dvar = acc_var[jc & 1];
        if (jc > 0) step_sync();
        issue_after(jc);
        const uint16_t* ops = L.buf[(slot + jc) & 1];
        dmu = f32x16{};
        dvar = f32x16{};
        if (jc > 0 && !mine) {
          // this half owns chunk jc - 1: its fold, in pieces between this chunk's products
          PairFold<kSecond, kDisp> f{acc_mu[(jc - 1) & 1], acc_var[(jc - 1) & 1], xs, jc - 1, lane,
                                     L.log2_n, L.log2_sigma, k};
          pair_products<kSecond>(ops, e0k, qb, q2h, q2l, dmu, dvar,
                                 [&](int dc) { f.piece(dc, m_run, l_run, st[(jc - 1) >> 1]); });
        } else {
          pair_products<kSecond>(ops, e0k, qb, q2h, q2l, dmu, dvar, [](int) {});
        }
        if (!mine) put_partial<kSecond>(xs, lane, dmu, dvar);
      }
    }
    if (nsteps == nstored) issue_next_item();
    if (nstored > 0) {
      // the last stored chunk c: its partner's products are in the slot after this
      // barrier; its owner (the half with KH == c & 1) holds its own in acc[KH]
      block_sync();
      const int c = nstored - 1;
      if (KH == (c & 1)) {
#pragma unroll
        for (int i = 0; i < 4; ++i) add_partial<kSecond>(xs, lane, i, acc_mu[KH], acc_var[KH]);
        float lg[16], val[16];
        chunk_logits<kSecond, kDisp>(acc_mu[KH], acc_var[KH], c, t, lane, L.log2_n, L.log2_sigma,
                                     k, lg, val);
        fold_row(lg, m_run, l_run);
#pragma unroll
        for (int e = 0; e < S / 2; ++e) {
          if (e == (c >> 1)) {
#pragma unroll
            for (int r = 0; r < 16; ++r) st[e][r] = kDisp ? val[r] : lg[r];
          }
        }
      }
    }
    // ---- chunks past S, first pass: the row state only
    for (int jc = S; jc < nchunks; ++jc) {
      const bool mine = KH == (jc & 1);
      f32x16 dmu = {}, dvar = {};
      step_sync();
      issue_after(jc);
      pair_products<kSecond>(L.buf[(slot + jc) & 1], e0k, qb, q2h, q2l, dmu, dvar, [](int) {});
      if (!mine) put_partial<kSecond>(xs, lane, dmu, dvar);
      block_sync();
      if (mine) {
#pragma unroll
        for (int i = 0; i < 4; ++i) add_partial<kSecond>(xs, lane, i, dmu, dvar);
        float lg[16], val[16];
        chunk_logits<kSecond, kDisp>(dmu, dvar, jc, t, lane, L.log2_n, L.log2_sigma, k, lg, val);
        fold_row(lg, m_run, l_run);
      }
    }


    // ---- each row's softmax maximum and sum: the two lane halves, then the two
    // halves of the workgroup (combined in the order KH 0, KH 1 by both)
    float inv_l;
    {
      const float om = xor32(m_run), ol = xor32(l_run);
      const float nm = fmaxf(m_run, om);
      float nl = 0.0f;
      if (nm != -INFINITY) {
        nl = (m_run == -INFINITY ? 0.0f : l_run * exp2_fast(m_run - nm)) +
             (om == -INFINITY ? 0.0f : ol * exp2_fast(om - nm));
      }
      if (half == 0) L.rowstate[KH][rg * 32 + col] = make_float2(nm, nl);
      block_sync();
      const float2 s0 = L.rowstate[0][rg * 32 + col], s1 = L.rowstate[1][rg * 32 + col];
      const float mm = fmaxf(s0.x, s1.x);
      float ll = 0.0f;
      if (mm != -INFINITY) {
        ll = (s0.x == -INFINITY ? 0.0f : s0.y * exp2_fast(s0.x - mm)) +
             (s1.x == -INFINITY ? 0.0f : s1.y * exp2_fast(s1.x - mm));
      }
      m_run = mm;
      // rows past the sequence end contribute nothing
      inv_l = (ll > 0.0f && row_ok) ? 1.0f / ll : 0.0f;
    }
#pragma unroll
    for (int jc = KH; jc < S; jc += 2) {
      if (jc < nstored) {
        float v[16];
#pragma unroll
        for (int r = 0; r < 16; ++r) v[r] = st[jc >> 1][r];
        chunk_sums(v, m_run, inv_l, jc, rg, lane, L.part);
      }
    }
    // ---- chunks past S, second pass: products again, the owner's sums
    for (int jc = nstored; jc < nchunks; ++jc) {
      const int sc = nchunks + (jc - nstored);
      const bool mine = KH == (jc & 1);
      f32x16 dmu = {}, dvar = {};
      step_sync();
      issue_after(sc);
      pair_products<kSecond>(L.buf[(slot + sc) & 1], e0k, qb, q2h, q2l, dmu, dvar, [](int) {});
      if (!mine) put_partial<kSecond>(xs, lane, dmu, dvar);
      block_sync();
      if (mine) {
#pragma unroll
        for (int i = 0; i < 4; ++i) add_partial<kSecond>(xs, lane, i, dmu, dvar);
        float lg[16], val[16];
        chunk_logits<kSecond, kDisp>(dmu, dvar, jc, t, lane, L.log2_n, L.log2_sigma, k, lg, val);
        if constexpr (kDisp) chunk_sums(val, m_run, inv_l, jc, rg, lane, L.part);
        else chunk_sums(lg, m_run, inv_l, jc, rg, lane, L.part);
      }
    }
    if (nsteps > nchunks) issue_next_item();

    block_sync();  // every wave's block sums are in part
    const float inv_rows = 1.0f / (float)min(kBlock, a.seq - t * kBlock);
    for (int j = tid; j < a.blocks; j += kPairThreads) {
      const float sc = j < t ? (L.part[0][j] + L.part[1][j] + L.part[2][j] + L.part[3][j]) * inv_rows
                             : 0.0f;
      a.score[b * a.ss_b + t * a.ss_t + j * a.ss_j + h * a.ss_h] = sc;
    }
    slot = (slot + nsteps) & 1;
  }
}

template <int SEL, int S>
__global__ __launch_bounds__(kPairThreads, 1) void selector_pair_kernel(SelArgs args) {
  constexpr bool kSecond = SEL != SPX_SELECTOR_MEAN_BALANCED;
  constexpr bool kDisp = SEL == SPX_SELECTOR_DISPERSION_MEAN;
  constexpr int kParts = kSecond ? 4 : 2;
  static_assert(S % 2 == 0, "stored chunks alternate between the two halves");

  // sized for the second-order selectors whatever SEL is (mean_balanced copies and
  // exchanges only the first half of each buffer and slot): the views index with
  // the full strides
  __shared__ __align__(16) uint16_t buf[2][4 * kSelPart];
  __shared__ __align__(16) uint16_t qbuf[kBlock * 128];
  __shared__ __align__(16) float xbuf[4][8 * 64 * 4];
  __shared__ float log2_n[kSelMaxBlocks];
  __shared__ float log2_sigma[kDisp ? kSelMaxBlocks : 1];
  __shared__ float part[4][kSelMaxBlocks];
  __shared__ float2 rowstate[2][kBlock];
  const PairLds L{buf, qbuf, xbuf, log2_n, log2_sigma, part, rowstate};

  {
    const int tid = threadIdx.x;
    for (int j = tid; j < args.blocks; j += kPairThreads) log2_n[j] = log2f((float)args.counts[j]);
    const int per_tile = args.batch * args.q_heads;
    const int item = xcd_item(blockIdx.x, 0, gridDim.x, per_tile);
    if (item < args.blocks * per_tile) {
      const int t = args.blocks - 1 - item / per_tile, bh = item % per_tile;
      const int b = bh / args.q_heads, h = bh % args.q_heads;
      dma_q<128, kPairThreads>(args, t, b, h, qbuf, tid);
      if (t > 0) {
        const int64_t bg_elems = (int64_t)args.chunks * kSelChunkElems;
        dma_chunk<kParts, kPairThreads>(
            args.ws + ((int64_t)b * args.kv_heads + h / (args.q_heads / args.kv_heads)) * bg_elems,
            buf[0], tid);
      }
    }
  }
  if (__builtin_amdgcn_readfirstlane((int)threadIdx.x >> 8) == 0) pair_waves<SEL, S, 0>(args, L);
  else pair_waves<SEL, S, 1>(args, L);
}

// ---------------------------------------------------------------------------
// head_dim 128, rows of up to 256 blocks: two items per workgroup.
//
// One persistent workgroup of eight waves per CU takes items (tile pair t, t - 1;
// batch; q head), heaviest first: waves 0-3 hold the 32-row groups of tile t,
// waves 4-7 those of tile t - 1, each wave with all 128 dims of its rows (no
// partial products to exchange). Both tiles read the same head's descriptor
// chunks, so every chunk copied into LDS serves eight waves, and each SIMD runs
// one wave of each tile: one wave's softmax and reduction issue beside the other's
// products. At two waves per SIMD the registers hold the logits of the first S
// chunks; a tile with more chunks forms the products of the rest a second time.
// Products of all 128 dims (eight k-steps) without a read-ahead register set: at
// two waves per SIMD the other wave covers the operand reads' latency.
template <bool kSecond>
__device__ __forceinline__ void duo_products(const uint16_t* ops, int e0, const bf16x8 (&qb)[8],
                                             const bf16x8 (&q2h)[8], const bf16x8 (&q2l)[8],
                                             f32x16& dmu, f32x16& dvar) {
#pragma unroll
  for (int dc = 0; dc < 8; ++dc) {
    const int off = e0 ^ (dc << 4);
    dmu = mfma32(as_bf16x8(*reinterpret_cast<const u32x4*>(ops + off)), qb[dc], dmu);
    dmu = mfma32(as_bf16x8(*reinterpret_cast<const u32x4*>(ops + kSelPart + off)), qb[dc], dmu);
    if constexpr (kSecond) {
      const bf16x8 vh = as_bf16x8(*reinterpret_cast<const u32x4*>(ops + 2 * kSelPart + off));
      const bf16x8 vl = as_bf16x8(*reinterpret_cast<const u32x4*>(ops + 3 * kSelPart + off));
      dvar = mfma32(vh, q2h[dc], dvar);
      dvar = mfma32(vl, q2h[dc], dvar);
      dvar = mfma32(vh, q2l[dc], dvar);
    }
  }
}

constexpr int kDuoThreads = 512;
constexpr int kDuoMaxBlocks = 256;

template <int SEL, int S>
__global__ __launch_bounds__(kDuoThreads, 1) void selector_duo_kernel(SelArgs args) {
  constexpr bool kSecond = SEL != SPX_SELECTOR_MEAN_BALANCED;
  constexpr bool kDisp = SEL == SPX_SELECTOR_DISPERSION_MEAN;
  constexpr int kParts = kSecond ? 4 : 2;

  __shared__ __align__(16) uint16_t buf[2][kParts * kSelPart];
  __shared__ __align__(16) uint16_t qbuf[2][kBlock * 128];  // tile t - it at qbuf[it]
  __shared__ float log2_n[kDuoMaxBlocks];
  __shared__ float log2_sigma[kDisp ? kDuoMaxBlocks : 1];
  __shared__ float part[2][4][kDuoMaxBlocks];

  // The two tiles' Q rows into qbuf (16-byte chunk c of row r at c ^ (r & 15));
  // rows outside [0, seq) clamped (their registers are zeroed, or unused when
  // t - 1 < 0).
  auto dma_q2 = [&](const SelArgs& a, int t, int b, int h, int tid) {
    const int w = tid >> 6;
    const uint32_t lds_base =
        (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) uint16_t*)&qbuf[0][0];
    const uint16_t* base = a.q + (int64_t)b * a.qs_b + (int64_t)h * a.qs_h;
#pragma unroll
    for (int i = 0; i < 2 * kBlock * 16 / kDuoThreads; ++i) {
      const int p = i * kDuoThreads + tid;
      const int it = p >> 11, r = (p >> 4) & 127, c = (p & 15) ^ (r & 15);
      const int64_t row = max(0, min((t - it) * kBlock + r, a.seq - 1));
      dma_gather16(base + row * a.qs_s + c * 8,
                   lds_base + (uint32_t)(i * kDuoThreads + w * 64) * 16u);
    }
  };

  {
    const int tid = threadIdx.x;
    for (int j = tid; j < args.blocks; j += kDuoThreads) log2_n[j] = log2f((float)args.counts[j]);
    const int per_tile = args.batch * args.q_heads;
    const int item = xcd_item(blockIdx.x, 0, gridDim.x, per_tile);
    if (item < (args.blocks + 1) / 2 * per_tile) {
      const int t = args.blocks - 1 - 2 * (item / per_tile), bh = item % per_tile;
      const int b = bh / args.q_heads, h = bh % args.q_heads;
      dma_q2(args, t, b, h, tid);
      if (t > 0)
        dma_chunk<kParts, kDuoThreads>(
            args.ws + ((int64_t)b * args.kv_heads + h / (args.q_heads / args.kv_heads)) *
                          args.chunks * kSelChunkElems,
            buf[0], tid);
    }
  }
  int slot = 0;  // buffer of the current item's first step

  for (int m = 0;; ++m) {
    // arguments re-read per item through an opaque pointer, the thread index through
    // an opaque copy: nothing derived from them is held across items
#if defined(__HIP_DEVICE_COMPILE__)
    const __attribute__((address_space(4))) SelArgs* ap =
        (const __attribute__((address_space(4))) SelArgs*)__builtin_amdgcn_kernarg_segment_ptr();
    asm volatile("" : "+s"(ap));
    const SelArgs a = *ap;
#else
    const SelArgs a = args;
#endif
    const int per_tile = a.batch * a.q_heads;
    const int n_items = (a.blocks + 1) / 2 * per_tile;
    const int item = xcd_item(blockIdx.x, m, gridDim.x, per_tile);
    if (item >= n_items) break;
    const int tid = opaque((int)threadIdx.x), lane = tid & 63;
    const int it = __builtin_amdgcn_readfirstlane(tid >> 8);  // tile t - it
    const int w = (tid >> 6) & 3;                              // row group
    const int col = lane & 31, half = lane >> 5;
    const int group = a.q_heads / a.kv_heads;
    const int64_t bg_elems = (int64_t)a.chunks * kSelChunkElems;
    const SelConsts k{a.scale * kLog2e, 0.5f * a.scale * a.scale * kLog2e, a.scale * a.scale};
    const int e0 = col * 128 + (((col >> 1) & 7) << 4) + ((half ^ (col & 1)) << 3);

    const int t = a.blocks - 1 - 2 * (item / per_tile), bh = item % per_tile;
    const int b = bh / a.q_heads, h = bh % a.q_heads, g = h / group;
    const int tile = t - it;                                   // this wave's tile (-1: none)
    const int nchunks = (t + kSelChunk - 1) / kSelChunk;       // the workgroup's steps: tile t
    const int nstored = min(nchunks, S);
    const int nsteps = nchunks + (nchunks - nstored);          // pass 1, then pass 2 past S
    const int my_chunks = tile > 0 ? (tile + kSelChunk - 1) / kSelChunk : 0;
    const uint16_t* src = a.ws + ((int64_t)b * a.kv_heads + g) * bg_elems;
    const int next = xcd_item(blockIdx.x, m + 1, gridDim.x, per_tile);

    auto issue_after = [&](int s) {
      if (s + 1 < nsteps) {
        const int s1 = s + 1;
        const int jc = s1 < nchunks ? s1 : nstored + (s1 - nchunks);
        dma_chunk<kParts, kDuoThreads>(src + (int64_t)jc * kSelChunkElems, buf[(slot + s1) & 1], tid);
      }
    };
    auto issue_next_item = [&]() {
      if (next < n_items) {
        const int nt = a.blocks - 1 - 2 * (next / per_tile), nbh = next % per_tile;
        const int nb = nbh / a.q_heads, nh = nbh % a.q_heads;
        dma_q2(a, nt, nb, nh, tid);
        if (nt > 0)
          dma_chunk<kParts, kDuoThreads>(a.ws + ((int64_t)nb * a.kv_heads + nh / group) * bg_elems,
                                         buf[(slot + nsteps) & 1], tid);
      }
    };
    auto step_sync = [&]() {
      asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
      block_sync();
    };

    step_sync();  // Q and the first chunk landed; the previous item's LDS reads are done
    const int64_t qrow = (int64_t)tile * kBlock + w * 32 + col;
    const bool row_ok = tile >= 0 && qrow < a.seq;
    bf16x8 qb[8], q2h[8], q2l[8];
    read_q<kSecond, 128>(qbuf[it], w, col, half, row_ok, qb, q2h, q2l);
    if (kDisp) {
      for (int j = tid; j < t; j += kDuoThreads)
        log2_sigma[j] = __log2f(a.sigma_v[((int64_t)b * a.blocks + j) * a.kv_heads + g]);
    }
    block_sync();  // the Q tiles are free for the next item's copy; log2_sigma visible
    if (nsteps == 0) issue_next_item();

    float m_run = -INFINITY, l_run = 0.0f;  // this lane's row state over its blocks
    float st[S][16] = {};                    // logits of the stored chunks
    f32x16 dmu = {}, dvar = {};

    // ---- stored chunks: products, then the fold (the other tile's wave on the
    // SIMD fills the matrix core meanwhile)
#pragma unroll
    for (int jc = 0; jc < S; ++jc) {
      if (jc < nstored) {
        if (jc > 0) step_sync();
        issue_after(jc);
        if (jc < my_chunks) {
          dmu = f32x16{};
          dvar = f32x16{};
          duo_products<kSecond>(buf[(slot + jc) & 1], e0, qb, q2h, q2l, dmu, dvar);
          float lg[16], val[16];
          chunk_logits<kSecond, kDisp>(dmu, dvar, jc, tile, lane, log2_n, log2_sigma, k, lg, val);
          fold_row(lg, m_run, l_run);
#pragma unroll
          for (int r = 0; r < 16; ++r) st[jc][r] = kDisp ? val[r] : lg[r];
        }
      }
    }
    // ---- chunks past S, first pass: the row state only
    for (int jc = S; jc < nchunks; ++jc) {
      step_sync();
      issue_after(jc);
      if (jc < my_chunks) {
        dmu = f32x16{};
        dvar = f32x16{};
        duo_products<kSecond>(buf[(slot + jc) & 1], e0, qb, q2h, q2l, dmu, dvar);
        float lg[16], val[16];
        chunk_logits<kSecond, kDisp>(dmu, dvar, jc, tile, lane, log2_n, log2_sigma, k, lg, val);
        fold_row(lg, m_run, l_run);
      }
    }
    if (nsteps == nchunks) issue_next_item();

    // ---- the row's softmax maximum and sum: merge the two lane halves
    float inv_l;
    {
      const float om = xor32(m_run), ol = xor32(l_run);
      const float nm = fmaxf(m_run, om);
      float nl = 0.0f;
      if (nm != -INFINITY) {
        nl = (m_run == -INFINITY ? 0.0f : l_run * exp2_fast(m_run - nm)) +
             (om == -INFINITY ? 0.0f : ol * exp2_fast(om - nm));
      }
      m_run = nm;
      // rows past the sequence end contribute nothing
      inv_l = (nl > 0.0f && row_ok) ? 1.0f / nl : 0.0f;
    }
#pragma unroll
    for (int jc = 0; jc < S; ++jc) {
      if (jc < nstored && jc < my_chunks) {
        float v[16];
#pragma unroll
        for (int r = 0; r < 16; ++r) v[r] = st[jc][r];
        chunk_sums(v, m_run, inv_l, jc, w, lane, part[it]);
      }
    }
    // ---- chunks past S, second pass: products again, then their sums
    for (int jc = nstored; jc < nchunks; ++jc) {
      const int sc = nchunks + (jc - nstored);
      step_sync();
      issue_after(sc);
      if (jc < my_chunks) {
        dmu = f32x16{};
        dvar = f32x16{};
        duo_products<kSecond>(buf[(slot + sc) & 1], e0, qb, q2h, q2l, dmu, dvar);
        float lg[16], val[16];
        chunk_logits<kSecond, kDisp>(dmu, dvar, jc, tile, lane, log2_n, log2_sigma, k, lg, val);
        if constexpr (kDisp) chunk_sums(val, m_run, inv_l, jc, w, lane, part[it]);
        else chunk_sums(lg, m_run, inv_l, jc, w, lane, part[it]);
      }
    }
    if (nsteps > nchunks) issue_next_item();

    block_sync();  // every wave's block sums are in part
    {
      // thread (tile t - i, block j): i = tid / 256, j = tid % 256 (blocks <= 256)
      const int i = tid >> 8, j = tid & 255, tt = t - i;
      if (tt >= 0 && j < a.blocks) {
        const float inv_rows = 1.0f / (float)min(kBlock, a.seq - tt * kBlock);
        const float sc = j < tt ? (part[i][0][j] + part[i][1][j] + part[i][2][j] + part[i][3][j]) * inv_rows
                                : 0.0f;
        a.score[b * a.ss_b + tt * a.ss_t + j * a.ss_j + h * a.ss_h] = sc;
      }
    }
    slot = (slot + nsteps) & 1;
  }
}

}  // namespace spx

using namespace spx;

static int64_t selector_chunks(int seq) { return (num_blocks(seq) + kSelChunk - 1) / kSelChunk; }

extern "C" int64_t spx_selector_workspace_bytes(int batch, int seq, int kv_heads, int head_dim) {
  if (batch <= 0 || seq <= 0 || kv_heads <= 0 || (head_dim != 128 && head_dim != 256)) return -1;
  return (int64_t)batch * kv_heads * selector_chunks(seq) * (head_dim / 128) * kSelChunkElems * 2;
}

namespace {

// Chunks whose logits a selector kernel keeps in AGPRs (16 per lane each): as many
// as the register file holds beside the kernel's other state without scratch.
constexpr int sel_store(int sel, int d, bool long_rows) {
  return d == 256 ? 4 : !long_rows ? 8 : sel == SPX_SELECTOR_DISPERSION_MEAN ? 10 : 12;
}

// Compute units of the current device (one persistent workgroup each).
int64_t cu_count() {
  static int per_device[64] = {};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  if (per_device[dev] == 0) {
    int cus = 0;
    if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
        cus < 1)
      cus = 256;
    per_device[dev] = cus;
  }
  return per_device[dev];
}

int run_selectors(const void* q, const int64_t* q_strides, const float* mean_k,
                  const float* var_k, const float* sigma_v, const int32_t* counts, int batch,
                  int seq, int q_heads, int kv_heads, int head_dim, int block_size, int selector,
                  float scale, void* workspace, float* score, const int64_t* score_strides,
                  void* stream) {
  SPX_REQUIRE(selector == SPX_SELECTOR_MEAN_BALANCED || selector == SPX_SELECTOR_CGF_MEAN ||
                  selector == SPX_SELECTOR_DISPERSION_MEAN,
              SPX_EINVAL, "unsupported selector id %d", selector);
  SPX_REQUIRE(head_dim == 128 || head_dim == 256, SPX_EUNSUPPORTED,
              "head_dim %d unsupported (128 or 256)", head_dim);
  SPX_REQUIRE(block_size == kBlock, SPX_EUNSUPPORTED, "block_size %d unsupported (only 128)", block_size);
  SPX_REQUIRE(batch > 0 && seq > 0 && q_heads > 0 && kv_heads > 0 && q_heads % kv_heads == 0,
              SPX_EINVAL, "bad shape");
  SPX_REQUIRE(q && q_strides && q_strides[3] == 1 && (reinterpret_cast<uintptr_t>(q) & 15) == 0 &&
                  q_strides[0] % 8 == 0 && q_strides[1] % 8 == 0 && q_strides[2] % 8 == 0,
              SPX_EINVAL, "q: null, misaligned or non-unit dim stride");
  SPX_REQUIRE(mean_k && counts && score && score_strides && workspace, SPX_EINVAL, "null pointer");
  SPX_REQUIRE((reinterpret_cast<uintptr_t>(mean_k) & 15) == 0 &&
                  (reinterpret_cast<uintptr_t>(var_k) & 15) == 0 &&
                  (reinterpret_cast<uintptr_t>(workspace) & 15) == 0,
              SPX_EINVAL, "mean_k / var_k / workspace must be 16-byte aligned");
  SPX_REQUIRE(selector == SPX_SELECTOR_MEAN_BALANCED || var_k, SPX_EINVAL, "var_k: null pointer");
  SPX_REQUIRE(selector != SPX_SELECTOR_DISPERSION_MEAN || sigma_v, SPX_EINVAL, "sigma_v: null pointer");
  const int blocks = num_blocks(seq);
  SPX_REQUIRE(blocks <= kSelMaxBlocks, SPX_EUNSUPPORTED, "seq %d exceeds %d blocks", seq, kSelMaxBlocks);
  hipStream_t st = static_cast<hipStream_t>(stream);
  const int chunks = (int)selector_chunks(seq);

  SplitArgs sa{};
  sa.mean_k = mean_k; sa.var_k = var_k;
  sa.ws = static_cast<uint16_t*>(workspace);
  sa.batch = batch; sa.kv_heads = kv_heads; sa.blocks = blocks; sa.chunks = chunks;
  sa.dim = head_dim;
  sa.second_order = selector != SPX_SELECTOR_MEAN_BALANCED;
  sa.mu_mul = 1.0f;
  sa.var_mul = 1.0f;
  const int64_t threads = (int64_t)batch * kv_heads * chunks * kSelChunk * (head_dim / 8);
  selector_split_kernel<<<(unsigned)((threads + 255) / 256), 256, 0, st>>>(sa);
  int rc = launch_status("selector_split");
  if (rc) return rc;

  SelArgs a{};
  a.q = static_cast<const uint16_t*>(q);
  a.qs_b = q_strides[0]; a.qs_s = q_strides[1]; a.qs_h = q_strides[2];
  a.ws = static_cast<const uint16_t*>(workspace);
  a.sigma_v = sigma_v; a.counts = counts;
  a.batch = batch; a.seq = seq; a.q_heads = q_heads; a.kv_heads = kv_heads; a.blocks = blocks;
  a.chunks = chunks;
  a.scale = scale;
  a.score = score;
  a.ss_b = score_strides[0]; a.ss_t = score_strides[1]; a.ss_j = score_strides[2];
  a.ss_h = score_strides[3];
  // persistent grids: a multiple of 8 workgroups (xcd_item), at most one per CU
  // and at most one per item rounded up to 8 (the spare ones find no item and exit)
  const int64_t items = (int64_t)blocks * batch * q_heads;
  auto grid_for = [](int64_t n) {
    const int64_t cus = std::max<int64_t>(8, cu_count() / 8 * 8);
    return (unsigned)std::min<int64_t>(cus, (n + 7) / 8 * 8);
  };
  const unsigned grid = grid_for(items);
  // Up to 8 chunks (256 blocks) at head_dim 128: mean_balanced in the duo kernel
  // (two tiles per workgroup, every chunk's logits in registers: 0.155 ms at 32K
  // against 0.211 ms in the pair kernel), cgf_mean and dispersion_mean in the pair
  // kernel (the q*q split leaves the duo kernel room for 3 chunks only, and the
  // products formed twice for the rest made it no faster: 0.308 / 0.369 ms against
  // 0.304 / 0.347 ms). Longer rows and head_dim 256: the one-wave-per-SIMD kernel,
  // its logits of sel_store(...) chunks in AGPRs and the products of the rest formed
  // twice (on 131072-token rows it ran 5.0-5.3 ms per cgf_mean layer against 5.6 ms
  // for the pair kernel with its unstored chunks in two-barrier steps).
  const bool long_rows = chunks > 8;
  const unsigned duo_grid = grid_for((int64_t)(blocks + 1) / 2 * batch * q_heads);
  switch (selector * 1000 + head_dim * 2 + (long_rows ? 1 : 0)) {
#define SPX_SEL_CASE(SEL, D)                                                      \
  case SEL * 1000 + D * 2 + 1:                                                    \
    selector_kernel<SEL, D, sel_store(SEL, D, true)><<<grid, kSelThreads, 0, st>>>(a);  \
    break;
#define SPX_PAIR_CASE(SEL)                                                        \
  case SEL * 1000 + 256:                                                          \
    selector_pair_kernel<SEL, 8><<<grid, kPairThreads, 0, st>>>(a);               \
    break;
#define SPX_D256_CASE(SEL)                                                        \
  case SEL * 1000 + 512:                                                          \
    selector_kernel<SEL, 256, sel_store(SEL, 256, false)><<<grid, kSelThreads, 0, st>>>(a); \
    break;
    case SPX_SELECTOR_MEAN_BALANCED * 1000 + 256:
      selector_duo_kernel<SPX_SELECTOR_MEAN_BALANCED, 8><<<duo_grid, kDuoThreads, 0, st>>>(a);
      break;
    SPX_PAIR_CASE(SPX_SELECTOR_CGF_MEAN)
    SPX_PAIR_CASE(SPX_SELECTOR_DISPERSION_MEAN)
    SPX_SEL_CASE(SPX_SELECTOR_MEAN_BALANCED, 128)
    SPX_SEL_CASE(SPX_SELECTOR_CGF_MEAN, 128)
    SPX_SEL_CASE(SPX_SELECTOR_DISPERSION_MEAN, 128)
    SPX_SEL_CASE(SPX_SELECTOR_MEAN_BALANCED, 256)
    SPX_SEL_CASE(SPX_SELECTOR_CGF_MEAN, 256)
    SPX_SEL_CASE(SPX_SELECTOR_DISPERSION_MEAN, 256)
    SPX_D256_CASE(SPX_SELECTOR_MEAN_BALANCED)
    SPX_D256_CASE(SPX_SELECTOR_CGF_MEAN)
    SPX_D256_CASE(SPX_SELECTOR_DISPERSION_MEAN)
#undef SPX_D256_CASE
#undef SPX_PAIR_CASE
#undef SPX_SEL_CASE
    default:
      SPX_REQUIRE(false, SPX_EINVAL, "unsupported selector %d / head_dim %d", selector, head_dim);
  }
  return launch_status("selector_scores");
}

}  // namespace

extern "C" int spx_selector_scores(const void* q, const int64_t* q_strides, const float* mean_k,
                                   const float* var_k, const float* sigma_v, const int32_t* counts,
                                   int batch, int seq, int q_heads, int kv_heads, int head_dim,
                                   int block_size, int selector, float scale, void* workspace,
                                   float* score, const int64_t* score_strides, void* stream) {
  return run_selectors(q, q_strides, mean_k, var_k, sigma_v, counts, batch, seq, q_heads,
                       kv_heads, head_dim, block_size, selector, scale, workspace, score,
                       score_strides, stream);
}

// ------------------------------------------------ no-allocation variant
//
// The split workspace of spx_selector_scores_noalloc lives in a file-scope device
// array, so the entry point needs no caller workspace and allocates nothing
// (callers under graph capture, tight serving loops). Every GPU holds its own copy
// of the array until the process ends; its device address is looked up once per
// device with hipGetSymbolAddress (the array's name in host code is only a
// host-side stand-in and must never reach a kernel). The split kernel rewrites
// every workspace entry a call reads (padded block rows as zeros), so nothing is
// cleared between calls; calls that overlap on one GPU race on the array.

constexpr int64_t kSelectorScratchBytes = 8ll << 20;   // B * Hkv * ceil(NB / 32) * (D / 128) <= 256

static __device__ __align__(256) uint8_t scratch[kSelectorScratchBytes];

namespace {

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mutex;
void* g_scratch[kMaxDevices] = {};

// Device address of `scratch` on the current device (looked up on first use).
int scratch_address(void* stream, void** out) {
  int device = -1;
  hipError_t e = hipGetDevice(&device);
  SPX_REQUIRE(e == hipSuccess, SPX_ELAUNCH, "hipGetDevice failed: %s", hipGetErrorString(e));
  SPX_REQUIRE(device >= 0 && device < kMaxDevices, SPX_EUNSUPPORTED,
              "device %d beyond the %d devices the scratch table covers", device, kMaxDevices);
  if (stream != nullptr) {
    int stream_device = -1;
    e = hipStreamGetDevice(static_cast<hipStream_t>(stream), &stream_device);
    SPX_REQUIRE(e == hipSuccess, SPX_EINVAL, "hipStreamGetDevice failed: %s", hipGetErrorString(e));
    SPX_REQUIRE(stream_device == device, SPX_EINVAL,
                "stream belongs to device %d but device %d is current", stream_device, device);
  }
  std::lock_guard<std::mutex> lock(g_scratch_mutex);
  if (g_scratch[device] == nullptr) {
    void* address = nullptr;
    e = hipGetSymbolAddress(&address, HIP_SYMBOL(scratch));
    SPX_REQUIRE(e == hipSuccess && address != nullptr, SPX_ELAUNCH,
                "hipGetSymbolAddress(scratch) failed on device %d: %s", device,
                hipGetErrorString(e));
    g_scratch[device] = address;
  }
  *out = g_scratch[device];
  return SPX_OK;
}

}  // namespace

extern "C" int spx_selector_scores_noalloc(const void* q, const int64_t* q_strides,
                                           const float* mean_k, const float* var_k,
                                           const float* sigma_v, const int32_t* counts, int batch,
                                           int seq, int q_heads, int kv_heads, int head_dim,
                                           int block_size, int selector, float scale, float* score,
                                           const int64_t* score_strides, void* stream) {
  const int64_t need = spx_selector_workspace_bytes(batch, seq, kv_heads, head_dim);
  SPX_REQUIRE(need > 0, SPX_EUNSUPPORTED,
              "bad or unsupported shape: batch %d seq %d kv_heads %d head_dim %d", batch, seq,
              kv_heads, head_dim);
  SPX_REQUIRE(need <= kSelectorScratchBytes, SPX_EUNSUPPORTED,
              "workspace of %lld bytes exceeds the %lld-byte static scratch (batch x kv_heads x "
              "ceil(blocks / 32) x head_dim / 128 must be at most 256); use spx_selector_scores "
              "with a caller workspace", (long long)need, (long long)kSelectorScratchBytes);
  void* workspace = nullptr;
  const int rc = scratch_address(stream, &workspace);
  if (rc) return rc;
  return run_selectors(q, q_strides, mean_k, var_k, sigma_v, counts, batch, seq, q_heads,
                       kv_heads, head_dim, block_size, selector, scale, workspace, score,
                       score_strides, stream);
}
