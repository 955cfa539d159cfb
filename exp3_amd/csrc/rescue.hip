// Rescue-token choice for the fp_v1_rescue methods (kernels.py:233-309).
//
// For query tile t, q head h and key block j < t, the rescue token is
// argmax_p qbar_{t,h} . k_{j,p} over the block's 128 positions, qbar the tile's mean
// query over its real rows (kernels.py:274-283, first position on ties as
// torch.argmax). Only blocks j <= NB - 2 can be history blocks of a later tile, and
// those are full.
//
// gfx950 design
//   * tile_mean_kernel: one thread per (q head, dim pair) and query tile, fp32 sums
//     over the tile's rows (coalesced 4-byte reads along the head's dims).
//   * rescue_choice_kernel: the token scores of block j against every later tile's
//     mean queries form a GEMM (128 tokens x 128 dims x (tiles, heads)); it runs on
//     bf16 MFMA with the key tile (bf16-exact) staged in LDS and the fp32 means
//     split exactly into three bf16 parts, followed by an in-register argmax.
#include "common.h"

namespace spx {

constexpr int kChoiceThreads = 256;  // four waves

struct MeanQArgs {
  const uint16_t* q;
  int64_t qs_b, qs_s, qs_h;
  float* qmean;  // [B, NB, Hq, D]
  int seq, q_heads, blocks;
};

// One workgroup per (b, tile, q head): thread (row group rg, 16-byte chunk c) loads
// its rows' chunk c (all loads in flight at once) and sums them in fp32; the row
// groups of a wave are combined by lane exchanges and the four waves in a fixed
// order through LDS.
template <int D>
__global__ __launch_bounds__(256) void tile_mean_kernel(MeanQArgs a) {
  constexpr int kChunks = D / 8;              // 16-byte chunks per row
  constexpr int kGroups = 256 / kChunks;      // row groups (16 at D = 128, 8 at D = 256)
  constexpr int kRowsPer = kBlock / kGroups;  // rows per thread
  const int t = blockIdx.x, h = blockIdx.y, b = blockIdx.z;
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int c = tid % kChunks, rg = tid / kChunks;
  const int row0 = t * kBlock;
  const int n = min(kBlock, a.seq - row0);
  const uint16_t* src = a.q + b * a.qs_b + (int64_t)row0 * a.qs_s + h * a.qs_h + c * 8;
  // unconditional loads (rows past the tile's end read its last row and are dropped
  // below): no branch separates the loads, so all of them are in flight at once
  u32x4 raw[kRowsPer];
#pragma unroll
  for (int i = 0; i < kRowsPer; ++i)
    raw[i] = *reinterpret_cast<const u32x4*>(src + (int64_t)min(rg * kRowsPer + i, n - 1) * a.qs_s);
  float s[8] = {};
#pragma unroll
  for (int i = 0; i < kRowsPer; ++i) {
    const bool ok = rg * kRowsPer + i < n;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      s[2 * e] += ok ? bf16_lo(raw[i][e]) : 0.0f;
      s[2 * e + 1] += ok ? bf16_hi(raw[i][e]) : 0.0f;
    }
  }
  // lanes of one wave holding the same chunk differ in the lane bits above the chunk
#pragma unroll
  for (int m = kChunks; m < 64; m <<= 1) {
#pragma unroll
    for (int e = 0; e < 8; ++e) s[e] += __shfl_xor(s[e], m);
  }
  __shared__ float part[4][D];
  if (lane < kChunks) {
#pragma unroll
    for (int e = 0; e < 8; ++e) part[w][c * 8 + e] = s[e];
  }
  block_sync();
  if (tid < D) {
    const float sum = part[0][tid] + part[1][tid] + part[2][tid] + part[3][tid];
    a.qmean[(((int64_t)b * a.blocks + t) * a.q_heads + h) * D + tid] = sum / (float)n;
  }
}

struct ChoiceArgs {
  const float* qmean;    // [B, NB, Hq, D]
  const uint16_t* kt;    // key tiles [B, Hkv, NB, 128, D] (swizzled)
  uint8_t* choice;       // [B, NB, NB, Hq]
  int batch, q_heads, kv_heads, blocks, group;
  int splits;            // workgroups sharing one (key block, kv group)'s columns
};

__device__ __forceinline__ bf16x8 pack_bf16x8(const float (&x)[8]) {
  u32x4 r;
#pragma unroll
  for (int e = 0; e < 4; ++e) r[e] = pack_bf16x2(x[2 * e], x[2 * e + 1]);
  return as_bf16x8(r);
}

// Workgroups (key block j, kv group g, split s, batch b): the (later tile, q head)
// columns of block j are dealt in 32-column groups over the splits workgroups of
// (j, g) and their four waves (group s * 4 + w, then every splits * 4-th), so the
// early key blocks, which have the most later tiles, are spread over as many
// workgroups as the latest ones need. The key tile of block j
// (pool layout: row = token, 16-byte chunk c of row r at c ^ (r & 15) for c < 16;
// at D = 256, chunk c < 32 at (c & 16) | ((c & 15) ^ (r & 15))) is staged in LDS once; its 128 token rows are the MFMA A operand (four 32-row tiles). The
// columns are the (later tile t, q head) pairs of the group, 32 per wave step; their
// fp32 mean queries are split exactly into three bf16 parts (hi + mid + lo), so
// three bf16 products per k-step give the fp32 dot products to ~2^-24 relative.
// Each lane then owns one column's 128 token scores (64 per lane half, in token
// order): a strict in-lane max keeps the first position, and the two halves merge
// with the lower position on equal scores (torch.argmax: first maximum).
// Four waves per SIMD at D = 128 (at most 128 registers each); at D = 256 the 64 KB
// key tile allows two workgroups per CU.
template <int D>
__global__ __launch_bounds__(kChoiceThreads, D == 128 ? 4 : 2) void rescue_choice_kernel(ChoiceArgs a) {
  const int j = blockIdx.x;
  const int g = blockIdx.y / a.splits, split = blockIdx.y % a.splits;
  const int b = blockIdx.z;
  const int tid = threadIdx.x;
  const int lane = tid & 63, w = tid >> 6;
  const int col = lane & 31, half = lane >> 5;
  // entries of tiles t <= j (no rescue token) are written as 0, by split 0
  if (split == 0) {
    for (int i = tid; i < (j + 1) * a.group; i += kChoiceThreads) {
      const int t = i / a.group, hh = i % a.group;
      a.choice[(((int64_t)b * a.blocks + t) * a.blocks + j) * a.q_heads + g * a.group + hh] = 0;
    }
  }
  const int ncols = a.group * (a.blocks - 1 - j);   // 0 for the last block
  const int ngroups = (ncols + 31) / 32;
  if (split * (kChoiceThreads / 64) >= ngroups) return;   // no column group here

  __shared__ __align__(16) uint16_t kt[kBlock * D];  // 32 KB (64 KB at D = 256)
  {
    const u32x4* src = reinterpret_cast<const u32x4*>(
        a.kt + (((int64_t)b * a.kv_heads + g) * a.blocks + j) * kBlock * D);
    u32x4* dst = reinterpret_cast<u32x4*>(kt);
    for (int i = tid; i < kBlock * D / 8; i += kChoiceThreads) dst[i] = src[i];
  }
  block_sync();

  // LDS element offset of token row (32 rt + col), chunk 2 dc + half:
  // (dc >> 3) * 128 + (base ^ ((dc & 7) << 4)), plus rt * 32 rows
  const int e0 = (((col >> 1) & 7) << 4) + ((half ^ (col & 1)) << 3);
  for (int grp = split * (kChoiceThreads / 64) + w; grp < ngroups;
       grp += a.splits * (kChoiceThreads / 64)) {
    const int c = grp * 32 + col;
    const bool cok = c < ncols;
    const int t = j + 1 + (cok ? c / a.group : 0);
    const int hh = cok ? c % a.group : 0;
    const float* qm = a.qmean + (((int64_t)b * a.blocks + t) * a.q_heads + g * a.group + hh) * D +
                      half * 8;
    f32x16 acc[4] = {};
    // four k-steps per iteration: their mean-query loads and splits are formed
    // shortly before their products instead of all being hoisted (which held 192
    // registers and allowed two waves per SIMD)
#pragma unroll 4
    for (int dc = 0; dc < D / 16; ++dc) {
      float x[8] = {};
      if (cok) {
        const f32x4 x0 = *reinterpret_cast<const f32x4*>(qm + dc * 16);
        const f32x4 x1 = *reinterpret_cast<const f32x4*>(qm + dc * 16 + 4);
#pragma unroll
        for (int e = 0; e < 4; ++e) { x[e] = x0[e]; x[4 + e] = x1[e]; }
      }
      float r1[8], r2[8];
      const bf16x8 hi = pack_bf16x8(x);
#pragma unroll
      for (int e = 0; e < 8; ++e) r1[e] = x[e] - (float)hi[e];
      const bf16x8 mid = pack_bf16x8(r1);
#pragma unroll
      for (int e = 0; e < 8; ++e) r2[e] = r1[e] - (float)mid[e];
      const bf16x8 lo = pack_bf16x8(r2);
      const int off = col * D + (dc >> 3) * 128 + (e0 ^ ((dc & 7) << 4));
#pragma unroll
      for (int rt = 0; rt < 4; ++rt) {
        const bf16x8 kr = as_bf16x8(*reinterpret_cast<const u32x4*>(kt + rt * 32 * D + off));
        acc[rt] = mfma32(kr, hi, acc[rt]);
        acc[rt] = mfma32(kr, mid, acc[rt]);
        acc[rt] = mfma32(kr, lo, acc[rt]);
      }
    }
    float best = -INFINITY;
    int pos = 0;
#pragma unroll
    for (int rt = 0; rt < 4; ++rt) {
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const float v = acc[rt][r];
        if (v > best) {
          best = v;
          pos = rt * 32 + mfma32_row(r, lane);
        }
      }
    }
    const float ob = __shfl_xor(best, 32);
    const int op = __shfl_xor(pos, 32);
    if (ob > best || (ob == best && op < pos)) pos = op;
    if (half == 0 && cok)
      a.choice[(((int64_t)b * a.blocks + t) * a.blocks + j) * a.q_heads + g * a.group + hh] =
          (uint8_t)pos;
  }
}

}  // namespace spx

using namespace spx;

extern "C" int spx_tile_mean_query(const void* q, const int64_t* q_strides, int batch, int seq,
                                   int q_heads, int head_dim, int block_size, float* qmean,
                                   void* stream) {
  SPX_REQUIRE(head_dim == kHeadDim || head_dim == 256, SPX_EUNSUPPORTED,
              "head_dim %d unsupported (128 or 256)", head_dim);
  SPX_REQUIRE(block_size == kBlock, SPX_EUNSUPPORTED, "block_size %d unsupported (only 128)",
              block_size);
  SPX_REQUIRE(batch > 0 && seq > 0 && q_heads > 0, SPX_EINVAL, "bad shape: batch %d seq %d heads %d",
              batch, seq, q_heads);
  SPX_REQUIRE(q && q_strides && qmean, SPX_EINVAL, "null pointer");
  SPX_REQUIRE(q_strides[3] == 1, SPX_EINVAL, "q: innermost (dim) stride must be 1");
  SPX_REQUIRE((reinterpret_cast<uintptr_t>(q) & 15) == 0 && q_strides[0] % 8 == 0 &&
                  q_strides[1] % 8 == 0 && q_strides[2] % 8 == 0,
              SPX_EINVAL, "q: base must be 16-byte aligned and batch / sequence / head strides multiples of 8 elements");
  MeanQArgs a{};
  a.q = static_cast<const uint16_t*>(q);
  a.qs_b = q_strides[0]; a.qs_s = q_strides[1]; a.qs_h = q_strides[2];
  a.qmean = qmean;
  a.seq = seq; a.q_heads = q_heads; a.blocks = num_blocks(seq);
  dim3 grid(a.blocks, q_heads, batch);
  if (head_dim == 256) tile_mean_kernel<256><<<grid, 256, 0, static_cast<hipStream_t>(stream)>>>(a);
  else tile_mean_kernel<kHeadDim><<<grid, 256, 0, static_cast<hipStream_t>(stream)>>>(a);
  return launch_status("tile_mean_query");
}

extern "C" int spx_rescue_choice(const float* qmean, const void* key_tiles, int batch, int seq,
                                 int q_heads, int kv_heads, int head_dim, int block_size,
                                 uint8_t* choice, void* stream) {
  SPX_REQUIRE(head_dim == kHeadDim || head_dim == 256, SPX_EUNSUPPORTED,
              "head_dim %d unsupported (128 or 256)", head_dim);
  SPX_REQUIRE(block_size == kBlock, SPX_EUNSUPPORTED, "block_size %d unsupported (only 128)",
              block_size);
  SPX_REQUIRE(batch > 0 && seq > 0 && q_heads > 0 && kv_heads > 0 && q_heads % kv_heads == 0,
              SPX_EINVAL, "bad shape: batch %d seq %d q_heads %d kv_heads %d", batch, seq, q_heads,
              kv_heads);
  SPX_REQUIRE(qmean && key_tiles && choice, SPX_EINVAL, "null pointer");
  SPX_REQUIRE((reinterpret_cast<uintptr_t>(key_tiles) & 15) == 0 &&
                  (reinterpret_cast<uintptr_t>(qmean) & 15) == 0,
              SPX_EINVAL, "key_tiles and qmean must be 16-byte aligned");
  ChoiceArgs a{};
  a.qmean = qmean;
  a.kt = static_cast<const uint16_t*>(key_tiles);
  a.choice = choice;
  a.batch = batch; a.q_heads = q_heads; a.kv_heads = kv_heads; a.blocks = num_blocks(seq);
  a.group = q_heads / kv_heads;
  // enough splits that the first key block's column groups come to about four per wave
  // (two per wave ran the same at d = 128 and 8 % slower at d = 256, where every
  // workgroup stages a 64 KB key tile)
  const int max_groups = (a.group * (a.blocks - 1) + 31) / 32;
  a.splits = std::max(1, std::min(16, (max_groups + 4 * (kChoiceThreads / 64) - 1) /
                                          (4 * (kChoiceThreads / 64))));
  hipStream_t st = static_cast<hipStream_t>(stream);
  dim3 grid(a.blocks, kv_heads * a.splits, batch);
  if (head_dim == 256) rescue_choice_kernel<256><<<grid, kChoiceThreads, 0, st>>>(a);
  else rescue_choice_kernel<kHeadDim><<<grid, kChoiceThreads, 0, st>>>(a);
  return launch_status("rescue_choice");
}
