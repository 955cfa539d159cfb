// Routing: V1 block scores, threshold / protected selection and index lists.
//
// V1 score (upstream/flashprefill_native_forward.py:89-175 + normalize_scores
// :410-417). One workgroup per (query tile t, q head h): four waves each hold 32
// query rows of Q in registers as the MFMA A operand and stream the bf16 block
// means Kbar_j (B operand, L2-resident, 256 B per block) in chunks of 32 blocks:
//     S[row][j] = q_row . Kbar_j          (v_mfma_f32_32x32x16_bf16, fp32 acc)
//     x = S * fp32(scale * log2 e)
// Row i of tile t is valid for block j iff i >= 128 (j + 1) - 1 and i < S. Each
// lane reduces its 16 rows of one block column to (max, sum 2^(x - max)) and
// merges with the other lane half; every wave walks all chunks on its own (the
// next chunk's Kbar operands load while the current one is reduced) and leaves its
// rows' partials in LDS, and after one barrier the four waves' partials are merged
// in a fixed order, giving M_tj and m_tj. The normalisation w_j = m_tj 2^(M_tj - max_j M_tj) / (sum_j w + 1e-9)
// runs in the same workgroup, so the raw scores never reach HBM.
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

template <int D>
__global__ __launch_bounds__(kRouteThreads) void v1_route_kernel(V1Args a) {
  constexpr int kSteps = D / 16;  // 16-dim MFMA k-steps
  const int per_tile = a.batch * a.q_heads;
  const int t = a.blocks - 1 - blockIdx.x / per_tile;  // heaviest tiles first
  const int bh = blockIdx.x % per_tile;
  const int b = bh / a.q_heads, h = bh % a.q_heads;
  const int g = h / (a.q_heads / a.kv_heads);
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int col = lane & 31, half = lane >> 5;

  __shared__ float blk_max[kMaxBlocks];
  __shared__ float blk_mass[kMaxBlocks];
  __shared__ float part_max[4][kMaxBlocks];   // per-wave (max, mass) of every block
  __shared__ float part_mass[4][kMaxBlocks];
  __shared__ float scratch[8];
  __shared__ int wave_counts[8];

  // Q rows as A operands: lane holds row (wave * 32 + col), dims dc*16 + 8*half + 0..7.
  const int row_in_tile = wave * 32 + col;
  const int64_t qrow = (int64_t)t * kBlock + row_in_tile;
  bf16x8 qa[kSteps];
  {
    const uint16_t* src = a.q + b * a.qs_b + qrow * a.qs_s + h * a.qs_h + half * 8;
    const bool ok = qrow < a.seq;
#pragma unroll
    for (int dc = 0; dc < kSteps; ++dc) {
      u32x4 raw = {0u, 0u, 0u, 0u};
      if (ok) raw = *reinterpret_cast<const u32x4*>(src + dc * 16);
      qa[dc] = as_bf16x8(raw);
    }
  }
  const uint16_t* kb_base = a.kbar + b * a.ms_b + g * a.ms_h + half * 8;
  auto load_kbar = [&](int jc, bf16x8 (&kb)[kSteps]) {
    const int j = jc * 32 + col;
    const bool ok = j < a.blocks;
#pragma unroll
    for (int dc = 0; dc < kSteps; ++dc) {
      u32x4 raw = {0u, 0u, 0u, 0u};
      if (ok) raw = *reinterpret_cast<const u32x4*>(kb_base + (int64_t)j * a.ms_j + dc * 16);
      kb[dc] = as_bf16x8(raw);
    }
  };

  // Each wave walks every chunk of 32 blocks on its own (no barrier inside the
  // loop; the next chunk's Kbar operands load while this one is reduced) and
  // leaves its 32 rows' (max, mass) per block in LDS; the four waves merge after.
  // (prefetch at D = 128 only: at D = 256 the second operand set costs occupancy)
  constexpr bool kPrefetch = D == 128;
  const int nchunks = (t + 1 + 31) / 32;
  bf16x8 kb_next[kSteps];
  if (kPrefetch && nchunks > 0) load_kbar(0, kb_next);
  for (int jc = 0; jc < nchunks; ++jc) {
    const int j = jc * 32 + col;  // this lane's block column
    f32x16 acc = {};
    {
      bf16x8 kb[kSteps];
      if (kPrefetch) {
#pragma unroll
        for (int dc = 0; dc < kSteps; ++dc) kb[dc] = kb_next[dc];
        if (jc + 1 < nchunks) load_kbar(jc + 1, kb_next);
      } else {
        load_kbar(jc, kb);
      }
#pragma unroll
      for (int dc = 0; dc < kSteps; ++dc) acc = mfma32(qa[dc], kb[dc], acc);
    }
    // acc[r] = S[row 8*(r/4) + 4*half + r%4 of this wave][block j]
    const int64_t key_end = (int64_t)(j + 1) * kBlock - 1;
    float xs[16];
    float mx = -INFINITY;
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int64_t i = (int64_t)t * kBlock + wave * 32 + mfma32_row(r, lane);
      const bool valid = i >= key_end && i < a.seq;
      const float x = acc[r] * a.scale_log2;
      xs[r] = valid ? x : -INFINITY;
      mx = fmaxf(mx, xs[r]);
    }
    float mass = 0.0f;
    if (mx != -INFINITY) {
#pragma unroll
      for (int r = 0; r < 16; ++r) mass += exp2_fast(xs[r] - mx);
    }
    // merge the two lane halves (rows 4*half + ...)
    {
      const float om = xor32(mx), os = xor32(mass);
      const float nm = fmaxf(mx, om);
      float merged = 0.0f;
      if (nm != -INFINITY) {
        merged = (mx == -INFINITY ? 0.0f : mass * exp2_fast(mx - nm)) +
                 (om == -INFINITY ? 0.0f : os * exp2_fast(om - nm));
      }
      mx = nm;
      mass = merged;
    }
    if (half == 0 && j < a.blocks) {
      part_max[wave][j] = mx;
      part_mass[wave][j] = mass;
    }
  }
  block_sync();
  for (int jj = tid; jj < min(nchunks * 32, a.blocks); jj += kRouteThreads) {
    float m = part_max[0][jj];
    for (int w = 1; w < 4; ++w) m = fmaxf(m, part_max[w][jj]);
    float s2 = 0.0f;
    if (m != -INFINITY) {
      for (int w = 0; w < 4; ++w) {
        const float pm = part_max[w][jj];
        if (pm != -INFINITY) s2 += part_mass[w][jj] * exp2_fast(pm - m);
      }
    }
    blk_max[jj] = m;
    blk_mass[jj] = s2;
  }
  block_sync();

  // normalize_scores over j <= t; j > t has M = -inf and contributes 0.
  float local = -INFINITY;
  for (int jj = tid; jj <= t; jj += kRouteThreads) local = fmaxf(local, blk_max[jj]);
  const float gmax = block_reduce_max(local, scratch);
  float wsum = 0.0f;
  for (int jj = tid; jj <= t; jj += kRouteThreads) {
    const float m = blk_max[jj];
    const float w = (m != -INFINITY) ? blk_mass[jj] * exp2_fast(m - gmax) : 0.0f;
    blk_mass[jj] = w;
    wsum += w;
  }
  const float total = block_reduce_sum(wsum, scratch) + 1e-9f;
  for (int jj = tid; jj < a.blocks; jj += kRouteThreads) {
    const float s = jj <= t ? blk_mass[jj] / total : 0.0f;
    blk_mass[jj] = s;
    if (a.score) a.score[b * a.ss_b + t * a.ss_t + jj * a.ss_j + h * a.ss_h] = s;
  }
  if (a.indices) {
    block_sync();
    SelectOut o;
    o.indices = a.indices;
    o.counts = a.counts;
    o.mask = a.mask;
    o.heads = a.q_heads;
    o.row_base = (((int64_t)b * a.blocks + t) * a.blocks) * a.q_heads + h;
    o.count_off = ((int64_t)b * a.blocks + t) * a.q_heads + h;
    select_row(blk_mass, t, a.sel, o, scratch, wave_counts);
  }
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
  a->q = static_cast<const uint16_t*>(q);
  a->qs_b = q_strides[0]; a->qs_s = q_strides[1]; a->qs_h = q_strides[2];
  a->kbar = static_cast<const uint16_t*>(mean_k);
  a->ms_b = mk_strides[0]; a->ms_j = mk_strides[1]; a->ms_h = mk_strides[2];
  a->batch = batch; a->seq = seq; a->q_heads = q_heads; a->kv_heads = kv_heads;
  a->blocks = blocks;
  a->scale_log2 = (float)((double)scale * 1.4426950408889634);
  return SPX_OK;
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
  const int grid = a.blocks * batch * q_heads;
  if (head_dim == 128)
    v1_route_kernel<128><<<grid, kRouteThreads, 0, static_cast<hipStream_t>(stream)>>>(a);
  else
    v1_route_kernel<256><<<grid, kRouteThreads, 0, static_cast<hipStream_t>(stream)>>>(a);
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
  const int grid = a.blocks * batch * q_heads;
  if (head_dim == 128)
    v1_route_kernel<128><<<grid, kRouteThreads, 0, static_cast<hipStream_t>(stream)>>>(a);
  else
    v1_route_kernel<256><<<grid, kRouteThreads, 0, static_cast<hipStream_t>(stream)>>>(a);
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
  const int grid = batch * query_blocks * heads;
  select_kernel<<<grid, kRouteThreads, 0, static_cast<hipStream_t>(stream)>>>(a);
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
