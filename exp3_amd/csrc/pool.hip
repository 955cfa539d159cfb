// Block pooling: one HBM pass over K and V per (key block, kv head).
//
// Produces any subset of
//   * bf16 block-mean K (upstream/flashprefill_native_forward.py:27-69, 420-442):
//     fp32 sum over the valid rows / valid count, rounded to bf16;
//   * fp32 descriptors (kernels.py:22-46): mean_k, var_k = max(0, E[k^2] - mean^2),
//     mean_v, sigma_v = sqrt(sum_d max(0, E[v^2] - mean_v^2)), block counts;
//   * attention tiles: the block's K rows and its V transposed to [dim][128 key
//     slots] (key permutation of value_slot_of_key), rows / keys past the sequence
//     end zero, each 128 x 128 bf16 tile stored with 16-byte chunk c of row r at
//     position c ^ (r & 15). The attention kernel copies a tile into LDS verbatim
//     (direct global->LDS loads) and reads MFMA operands bank-conflict free.
//
// Bandwidth-bound: each workgroup streams a 128 x D bf16 K tile and V tile with
// 16-byte loads (each row is 2 D contiguous bytes), reduces columns in registers,
// across lanes and across the four waves through LDS. The V transpose stages one
// 64-key half of the rows in LDS at a time (the value slot permutation keeps slots
// 0-63 on keys 0-63), 25 KB of LDS per workgroup at D = 128: four workgroups per
// CU, so a 32K-token layer's 1020 workgroups run in one round.
//
// Head dim 256 (Qwen3.5 full-attention layers): the same pass; key tiles keep the
// [128 keys][256 dims] layout (chunk c of row r at c ^ (r & 15), c < 32), value tiles
// are four 32-key sub-blocks [256 dims][32 slots] (16 KB each, the d = 256 attention
// kernel's LDS image) with 16-byte chunk c of dim row d at c ^ ((d >> 2) & 3).
#include "common.h"

namespace spx {

struct PoolArgs {
  const uint16_t* k;
  int64_t ks_b, ks_s, ks_h;
  const uint16_t* v;
  int64_t vs_b, vs_s, vs_h;
  int batch, seq, kv_heads, blocks;
  uint16_t* mean_k_bf16;  // [B, NB, Hkv, D]
  float* mean_k;          // [B, NB, Hkv, D]
  float* mean_v;
  float* var_k;
  float* sigma_v;  // [B, NB, Hkv]
  int32_t* counts;  // [NB]
  uint16_t* key_tiles;    // [B, Hkv, NB, 128, D]
  uint16_t* value_tiles;  // [B, Hkv, NB, D, 128]
};

constexpr int kPoolThreads = 256;

__device__ __forceinline__ void accumulate8(const u32x4& raw, float* sum, float* sq) {
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    const float a = bf16_lo(raw[e]);
    const float b = bf16_hi(raw[e]);
    sum[2 * e] += a;
    sq[2 * e] = fmaf(a, a, sq[2 * e]);
    sum[2 * e + 1] += b;
    sq[2 * e + 1] = fmaf(b, b, sq[2 * e + 1]);
  }
}

// Sum a per-lane array of 8 floats over the row groups of a wave: lanes that differ
// in bits 4 and 5 (D = 128: 16 chunks per row) or in bit 5 (D = 256: 32 chunks).
template <int D>
__device__ __forceinline__ void reduce_row_groups(float* x) {
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    if (D == 128) x[e] += __shfl_xor(x[e], 16);
    x[e] += __shfl_xor(x[e], 32);
  }
}

template <int D, bool DO_K, bool DO_V, bool DO_TILES>
__global__ __launch_bounds__(kPoolThreads) void pool_kernel(PoolArgs a) {
  constexpr int kChunks = D / 8;                    // 16-byte chunks per row
  constexpr int kRowsPer = kBlock * kChunks / kPoolThreads;  // rows per row group
  constexpr int kVPitch = D + 2;                    // LDS row pitch (bf16) of staged V
  const int j = blockIdx.x;
  const int b = blockIdx.y / a.kv_heads;
  const int g = blockIdx.y % a.kv_heads;
  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = tid >> 6;
  const int c = tid & (kChunks - 1);  // 8-dim chunk
  const int rg = tid / kChunks;       // row group: rows rg * kRowsPer + i
  const int n = min(kBlock, a.seq - j * kBlock);

  __shared__ float part[4][4][D];                          // [quantity][wave][dim]
  __shared__ __align__(16) uint16_t vrows[kBlock / 2 * kVPitch];  // staged V rows, one half at a time
  __shared__ float sig_part[D / 64];

  float sk[8] = {}, qk[8] = {}, sv[8] = {}, qv[8] = {};
  const uint16_t* kbase = a.k + b * a.ks_b + g * a.ks_h + (int64_t)c * 8;
  const uint16_t* vbase = a.v + b * a.vs_b + g * a.vs_h + (int64_t)c * 8;
  const int64_t tile_off = ((((int64_t)b * a.kv_heads + g) * a.blocks + j) * kBlock) * D;
  u32x4 vraw[kRowsPer];   // this thread's V rows (all in one half of the block)

#pragma unroll
  for (int i = 0; i < kRowsPer; ++i) {
    const int row = rg * kRowsPer + i;
    const bool valid = row < n;
    const int64_t token = (int64_t)j * kBlock + row;
    if (DO_K || DO_TILES) {
      u32x4 raw = {0u, 0u, 0u, 0u};
      if (valid) raw = *reinterpret_cast<const u32x4*>(kbase + token * a.ks_s);
      if (DO_K && valid) accumulate8(raw, sk, qk);
      if (DO_TILES)
        *reinterpret_cast<u32x4*>(a.key_tiles + tile_off + row * D + ((c ^ (row & 15)) << 3)) = raw;
    }
    if (DO_V || DO_TILES) {
      u32x4 raw = {0u, 0u, 0u, 0u};
      if (valid) raw = *reinterpret_cast<const u32x4*>(vbase + token * a.vs_s);
      if (DO_V && valid) accumulate8(raw, sv, qv);
      if (DO_TILES) vraw[i] = raw;
    }
  }

  if (DO_K) { reduce_row_groups<D>(sk); reduce_row_groups<D>(qk); }
  if (DO_V) { reduce_row_groups<D>(sv); reduce_row_groups<D>(qv); }
  if (lane < kChunks) {
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const int d = c * 8 + e;
      if (DO_K) { part[0][wave][d] = sk[e]; part[1][wave][d] = qk[e]; }
      if (DO_V) { part[2][wave][d] = sv[e]; part[3][wave][d] = qv[e]; }
    }
  }
  block_sync();

  if (tid < D) {
    const int d = tid;
    const float count = (float)n;
    const int64_t o = (((int64_t)b * a.blocks + j) * a.kv_heads + g) * D + d;
    if (DO_K) {
      const float s = part[0][0][d] + part[0][1][d] + part[0][2][d] + part[0][3][d];
      const float s2 = part[1][0][d] + part[1][1][d] + part[1][2][d] + part[1][3][d];
      const float mean = s / count;
      if (a.mean_k_bf16) a.mean_k_bf16[o] = to_bf16_bits(mean);
      if (a.mean_k) a.mean_k[o] = mean;
      if (a.var_k) a.var_k[o] = fmaxf(s2 / count - mean * mean, 0.0f);
    }
    if (DO_V) {
      const float s = part[2][0][d] + part[2][1][d] + part[2][2][d] + part[2][3][d];
      const float s2 = part[3][0][d] + part[3][1][d] + part[3][2][d] + part[3][3][d];
      const float mean = s / count;
      const float var = fmaxf(s2 / count - mean * mean, 0.0f);
      if (a.mean_v) a.mean_v[o] = mean;
      if (a.sigma_v) {
        const float total = wave_sum(var);
        if ((tid & 63) == 0) sig_part[tid >> 6] = total;
      }
    }
  }
  if (a.counts && blockIdx.y == 0 && tid == 0) a.counts[j] = n;

  if (DO_TILES) {
    // Transposed write-out: thread -> (dim row d, 8-slot chunk gc); each gathers the
    // 8 keys of its slots from the staged rows and stores 16 bytes at the swizzled
    // chunk position (D = 128: [dim][128 slots], chunk gc ^ (d & 15); D = 256: sub-block
    // gc / 4 of [dim][32 slots], chunk (gc & 3) ^ ((d >> 2) & 3)).
    uint16_t* tile = a.value_tiles + tile_off;
    const int my_half = rg * kRowsPer / (kBlock / 2);
#pragma unroll
    for (int hh = 0; hh < 2; ++hh) {
      if (my_half == hh) {
#pragma unroll
        for (int i = 0; i < kRowsPer; ++i) {
          const int row = rg * kRowsPer + i - hh * (kBlock / 2);
          uint32_t* dst = reinterpret_cast<uint32_t*>(vrows + row * kVPitch + c * 8);
#pragma unroll
          for (int e = 0; e < 4; ++e) dst[e] = vraw[i][e];
        }
      }
      block_sync();
#pragma unroll
      for (int i = 0; i < 8 * D / kPoolThreads; ++i) {
        const int id = tid + kPoolThreads * i;  // 0 .. 8 D - 1
        const int d = id >> 3;                  // dim row of the tile
        const int chunk = hh * 8 + (id & 7);    // slots chunk * 8 .. chunk * 8 + 7 (keys of this half)
        uint32_t w[4];
#pragma unroll
        for (int m = 0; m < 8; m += 2) {
          const int s0 = chunk * 8 + m;
          // slot -> key: chunk16 * 16 + 4 * half + (m % 4) + 8 * (m / 4)
          const int c16 = s0 >> 4, half = (s0 >> 3) & 1, mm = s0 & 7;
          const int key0 = c16 * 16 + 4 * half + (mm & 3) + 8 * (mm >> 2) - hh * (kBlock / 2);
          const uint32_t lo = vrows[key0 * kVPitch + d];
          const uint32_t hi = vrows[(key0 + 1) * kVPitch + d];
          w[m >> 1] = lo | (hi << 16);
        }
        uint16_t* dst;
        if (D == 128)
          dst = tile + d * kBlock + ((chunk ^ (d & 15)) << 3);
        else
          dst = tile + (chunk >> 2) * (D * 32) + d * 32 + (((chunk & 3) ^ ((d >> 2) & 3)) << 3);
        *reinterpret_cast<u32x4*>(dst) = u32x4{w[0], w[1], w[2], w[3]};
      }
      if (hh == 0) block_sync();   // every read of the first half is done
    }
  }
  if (DO_V) {
    block_sync();
    if (a.sigma_v && tid == 0) {
      float total = 0.0f;
#pragma unroll
      for (int x = 0; x < D / 64; ++x) total += sig_part[x];
      a.sigma_v[((int64_t)b * a.blocks + j) * a.kv_heads + g] = sqrtf(total);
    }
  }
}

}  // namespace spx

using namespace spx;

template <int D>
static void launch_pool(int variant, dim3 grid, hipStream_t st, const PoolArgs& a) {
  switch (variant) {
    case 0: pool_kernel<D, false, false, false><<<grid, kPoolThreads, 0, st>>>(a); break;
    case 1: pool_kernel<D, false, false, true><<<grid, kPoolThreads, 0, st>>>(a); break;
    case 2: pool_kernel<D, false, true, false><<<grid, kPoolThreads, 0, st>>>(a); break;
    case 3: pool_kernel<D, false, true, true><<<grid, kPoolThreads, 0, st>>>(a); break;
    case 4: pool_kernel<D, true, false, false><<<grid, kPoolThreads, 0, st>>>(a); break;
    case 5: pool_kernel<D, true, false, true><<<grid, kPoolThreads, 0, st>>>(a); break;
    case 6: pool_kernel<D, true, true, false><<<grid, kPoolThreads, 0, st>>>(a); break;
    default: pool_kernel<D, true, true, true><<<grid, kPoolThreads, 0, st>>>(a); break;
  }
}

static int check_tensor4(const char* name, const void* p, const int64_t* st) {
  SPX_REQUIRE(p != nullptr && st != nullptr, SPX_EINVAL, "%s: null pointer", name);
  SPX_REQUIRE(st[3] == 1, SPX_EINVAL, "%s: innermost (dim) stride must be 1", name);
  SPX_REQUIRE((reinterpret_cast<uintptr_t>(p) & 15) == 0, SPX_EINVAL,
              "%s: base pointer must be 16-byte aligned", name);
  SPX_REQUIRE(st[0] % 8 == 0 && st[1] % 8 == 0 && st[2] % 8 == 0, SPX_EINVAL,
              "%s: batch / sequence / head strides must be multiples of 8 elements", name);
  return SPX_OK;
}

extern "C" int spx_block_pool(const void* k, const int64_t* k_strides, const void* v,
                              const int64_t* v_strides, int batch, int seq, int kv_heads,
                              int head_dim, int block_size, void* mean_k_bf16, float* mean_k,
                              float* mean_v, float* var_k, float* sigma_v, int32_t* counts,
                              void* key_tiles, void* value_tiles, void* stream) {
  SPX_REQUIRE(head_dim == 128 || head_dim == 256, SPX_EUNSUPPORTED,
              "head_dim %d unsupported (128 or 256)", head_dim);
  SPX_REQUIRE(block_size == kBlock, SPX_EUNSUPPORTED, "block_size %d unsupported (only 128)", block_size);
  SPX_REQUIRE(batch > 0 && seq > 0 && kv_heads > 0, SPX_EINVAL,
              "batch, seq and kv_heads must be positive (got %d, %d, %d)", batch, seq, kv_heads);
  SPX_REQUIRE((key_tiles == nullptr) == (value_tiles == nullptr), SPX_EINVAL,
              "key_tiles and value_tiles are produced together");
  const bool do_k = mean_k_bf16 || mean_k || var_k;
  const bool do_v = mean_v || sigma_v;
  const bool do_tiles = value_tiles != nullptr;
  if (do_k || do_tiles) { int e = check_tensor4("k", k, k_strides); if (e) return e; }
  if (do_v || do_tiles) { int e = check_tensor4("v", v, v_strides); if (e) return e; }
  if (do_tiles) {
    SPX_REQUIRE((reinterpret_cast<uintptr_t>(key_tiles) & 15) == 0 &&
                    (reinterpret_cast<uintptr_t>(value_tiles) & 15) == 0,
                SPX_EINVAL, "key_tiles / value_tiles must be 16-byte aligned");
  }
  if (!do_k && !do_v && !do_tiles && !counts) return SPX_OK;
  PoolArgs a{};
  a.k = static_cast<const uint16_t*>(k);
  if (do_k || do_tiles) { a.ks_b = k_strides[0]; a.ks_s = k_strides[1]; a.ks_h = k_strides[2]; }
  a.v = static_cast<const uint16_t*>(v);
  if (do_v || do_tiles) { a.vs_b = v_strides[0]; a.vs_s = v_strides[1]; a.vs_h = v_strides[2]; }
  a.batch = batch; a.seq = seq; a.kv_heads = kv_heads; a.blocks = num_blocks(seq);
  a.mean_k_bf16 = static_cast<uint16_t*>(mean_k_bf16);
  a.mean_k = mean_k; a.mean_v = mean_v; a.var_k = var_k; a.sigma_v = sigma_v;
  a.counts = counts;
  a.key_tiles = static_cast<uint16_t*>(key_tiles);
  a.value_tiles = static_cast<uint16_t*>(value_tiles);
  dim3 grid(a.blocks, batch * kv_heads);
  hipStream_t st = static_cast<hipStream_t>(stream);
  const int variant = (do_k ? 4 : 0) | (do_v ? 2 : 0) | (do_tiles ? 1 : 0);
  if (head_dim == 128) launch_pool<128>(variant, grid, st, a);
  else launch_pool<256>(variant, grid, st, a);
  return launch_status("block_pool");
}

extern "C" int spx_block_mean_k(const void* k, const int64_t* k_strides, int batch, int seq,
                                int kv_heads, int head_dim, int block_size, void* mean_k,
                                void* stream) {
  SPX_REQUIRE(mean_k != nullptr, SPX_EINVAL, "mean_k: null pointer");
  return spx_block_pool(k, k_strides, nullptr, nullptr, batch, seq, kv_heads, head_dim,
                        block_size, mean_k, nullptr, nullptr, nullptr, nullptr, nullptr,
                        nullptr, nullptr, stream);
}

extern "C" int spx_block_descriptors(const void* k, const int64_t* k_strides, const void* v,
                                     const int64_t* v_strides, int batch, int seq, int kv_heads,
                                     int head_dim, int block_size, float* mean_k, float* mean_v,
                                     float* var_k, float* sigma_v, int32_t* counts, void* stream) {
  SPX_REQUIRE(mean_k && mean_v && var_k && sigma_v && counts, SPX_EINVAL,
              "block_descriptors: every output must be given");
  return spx_block_pool(k, k_strides, v, v_strides, batch, seq, kv_heads, head_dim, block_size,
                        nullptr, mean_k, mean_v, var_k, sigma_v, counts, nullptr, nullptr, stream);
}
