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
//   * rescue_choice_kernel: one workgroup per (key block j, kv group), one thread
//     per token holding its key row in fp32 registers (read once from the key
//     tile, which is already in the K layout); for every later tile t the group's
//     mean queries are staged in LDS once and read by all threads as broadcasts,
//     each token's dot products being plain fp32 FMAs. The argmax is a
//     64-bit max over (order-preserving score bits, 127 - position) across the
//     block, which also picks the first position on ties.
#include "common.h"

namespace spx {

constexpr int kMaxGroup = 8;

struct MeanQArgs {
  const uint16_t* q;
  int64_t qs_b, qs_s, qs_h;
  float* qmean;  // [B, NB, Hq, D]
  int seq, q_heads, blocks;
};

__global__ __launch_bounds__(256) void tile_mean_kernel(MeanQArgs a) {
  const int t = blockIdx.x;
  const int b = blockIdx.z;
  const int idx = blockIdx.y * 256 + threadIdx.x;
  if (idx >= a.q_heads * (kHeadDim / 2)) return;
  const int h = idx / (kHeadDim / 2), d2 = idx % (kHeadDim / 2);
  const int row0 = t * kBlock;
  const int n = min(kBlock, a.seq - row0);
  const uint16_t* src = a.q + b * a.qs_b + (int64_t)row0 * a.qs_s + h * a.qs_h + 2 * d2;
  float s0 = 0.0f, s1 = 0.0f;
  for (int r = 0; r < n; ++r) {
    const uint32_t w = *reinterpret_cast<const uint32_t*>(src + (int64_t)r * a.qs_s);
    s0 += bf16_lo(w);
    s1 += bf16_hi(w);
  }
  const float count = (float)n;
  float* dst = a.qmean + (((int64_t)b * a.blocks + t) * a.q_heads + h) * kHeadDim + 2 * d2;
  dst[0] = s0 / count;
  dst[1] = s1 / count;
}

struct ChoiceArgs {
  const float* qmean;    // [B, NB, Hq, D]
  const uint16_t* kt;    // key tiles [B, Hkv, NB, 128, D] (swizzled)
  uint8_t* choice;       // [B, NB, NB, Hq]
  int batch, q_heads, kv_heads, blocks, group;
};

// float -> uint32 whose unsigned order is the float order (non-NaN values)
__device__ __forceinline__ uint32_t order_key(float x) {
  const uint32_t u = __float_as_uint(x);
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

__global__ __launch_bounds__(kBlock) void rescue_choice_kernel(ChoiceArgs a) {
  const int j = blockIdx.x;
  const int g = blockIdx.y;
  const int b = blockIdx.z;
  const int tok = threadIdx.x;
  const int lane = tok & 63, w = tok >> 6;
  // entries of tiles t <= j (no rescue token) are written as 0
  for (int i = tok; i < (j + 1) * a.group; i += kBlock) {
    const int t = i / a.group, hh = i % a.group;
    a.choice[(((int64_t)b * a.blocks + t) * a.blocks + j) * a.q_heads + g * a.group + hh] = 0;
  }
  if (j >= a.blocks - 1) return;  // no later tile

  float kf[kHeadDim];
  {
    const uint16_t* row =
        a.kt + ((((int64_t)b * a.kv_heads + g) * a.blocks + j) * kBlock + tok) * kHeadDim;
#pragma unroll
    for (int c = 0; c < kHeadDim / 8; ++c) {
      const u32x4 raw = *reinterpret_cast<const u32x4*>(row + ((c ^ (tok & 15)) << 3));
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        kf[8 * c + 2 * e] = bf16_lo(raw[e]);
        kf[8 * c + 2 * e + 1] = bf16_hi(raw[e]);
      }
    }
  }

  __shared__ __align__(16) float qs[kMaxGroup * kHeadDim];
  __shared__ uint64_t best[2][kMaxGroup];
  for (int t = j + 1; t < a.blocks; ++t) {
    const float* qm = a.qmean + (((int64_t)b * a.blocks + t) * a.q_heads + g * a.group) * kHeadDim;
    for (int i = tok; i < a.group * kHeadDim; i += kBlock) qs[i] = qm[i];
    block_sync();
    for (int hh = 0; hh < a.group; ++hh) {
      float s = 0.0f;
#pragma unroll
      for (int d = 0; d < kHeadDim; ++d) s = fmaf(qs[hh * kHeadDim + d], kf[d], s);
      uint64_t key = ((uint64_t)order_key(s) << 32) | (uint32_t)(kBlock - 1 - tok);
#pragma unroll
      for (int off = 32; off >= 1; off >>= 1) {
        const uint32_t lo = __shfl_xor((uint32_t)key, off);
        const uint32_t hi = __shfl_xor((uint32_t)(key >> 32), off);
        const uint64_t other = ((uint64_t)hi << 32) | lo;
        key = other > key ? other : key;
      }
      if (lane == 0) best[w][hh] = key;
    }
    block_sync();
    if (tok < a.group) {
      const uint64_t k0 = best[0][tok], k1 = best[1][tok];
      const uint64_t k = k0 > k1 ? k0 : k1;
      const int pos = kBlock - 1 - (int)(k & 0xffffffffu);
      a.choice[(((int64_t)b * a.blocks + t) * a.blocks + j) * a.q_heads + g * a.group + tok] =
          (uint8_t)pos;
    }
  }
}

}  // namespace spx

using namespace spx;

extern "C" int spx_tile_mean_query(const void* q, const int64_t* q_strides, int batch, int seq,
                                   int q_heads, int head_dim, int block_size, float* qmean,
                                   void* stream) {
  SPX_REQUIRE(head_dim == kHeadDim, SPX_EUNSUPPORTED, "head_dim %d unsupported (only 128)", head_dim);
  SPX_REQUIRE(block_size == kBlock, SPX_EUNSUPPORTED, "block_size %d unsupported (only 128)",
              block_size);
  SPX_REQUIRE(batch > 0 && seq > 0 && q_heads > 0, SPX_EINVAL, "bad shape: batch %d seq %d heads %d",
              batch, seq, q_heads);
  SPX_REQUIRE(q && q_strides && qmean, SPX_EINVAL, "null pointer");
  SPX_REQUIRE(q_strides[3] == 1, SPX_EINVAL, "q: innermost (dim) stride must be 1");
  SPX_REQUIRE((reinterpret_cast<uintptr_t>(q) & 3) == 0 && q_strides[0] % 2 == 0 &&
                  q_strides[1] % 2 == 0 && q_strides[2] % 2 == 0,
              SPX_EINVAL, "q: base and strides must keep dim pairs 4-byte aligned");
  MeanQArgs a{};
  a.q = static_cast<const uint16_t*>(q);
  a.qs_b = q_strides[0]; a.qs_s = q_strides[1]; a.qs_h = q_strides[2];
  a.qmean = qmean;
  a.seq = seq; a.q_heads = q_heads; a.blocks = num_blocks(seq);
  dim3 grid(a.blocks, (q_heads * (kHeadDim / 2) + 255) / 256, batch);
  tile_mean_kernel<<<grid, 256, 0, static_cast<hipStream_t>(stream)>>>(a);
  return launch_status("tile_mean_query");
}

extern "C" int spx_rescue_choice(const float* qmean, const void* key_tiles, int batch, int seq,
                                 int q_heads, int kv_heads, int head_dim, int block_size,
                                 uint8_t* choice, void* stream) {
  SPX_REQUIRE(head_dim == kHeadDim, SPX_EUNSUPPORTED, "head_dim %d unsupported (only 128)", head_dim);
  SPX_REQUIRE(block_size == kBlock, SPX_EUNSUPPORTED, "block_size %d unsupported (only 128)",
              block_size);
  SPX_REQUIRE(batch > 0 && seq > 0 && q_heads > 0 && kv_heads > 0 && q_heads % kv_heads == 0,
              SPX_EINVAL, "bad shape: batch %d seq %d q_heads %d kv_heads %d", batch, seq, q_heads,
              kv_heads);
  SPX_REQUIRE(q_heads / kv_heads <= kMaxGroup, SPX_EUNSUPPORTED,
              "more than %d q heads per kv head", kMaxGroup);
  SPX_REQUIRE(qmean && key_tiles && choice, SPX_EINVAL, "null pointer");
  SPX_REQUIRE((reinterpret_cast<uintptr_t>(key_tiles) & 15) == 0, SPX_EINVAL,
              "key_tiles must be 16-byte aligned");
  ChoiceArgs a{};
  a.qmean = qmean;
  a.kt = static_cast<const uint16_t*>(key_tiles);
  a.choice = choice;
  a.batch = batch; a.q_heads = q_heads; a.kv_heads = kv_heads; a.blocks = num_blocks(seq);
  a.group = q_heads / kv_heads;
  hipStream_t st = static_cast<hipStream_t>(stream);
  dim3 grid(a.blocks, kv_heads, batch);
  rescue_choice_kernel<<<grid, kBlock, 0, st>>>(a);
  return launch_status("rescue_choice");
}
