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
//   * selector_kernel: one workgroup per (tile, q head), four waves of 32 query
//     rows holding Q (and, at D = 128, the q*q hi/lo split) in registers as MFMA B
//     operands; at D = 256 the split is formed from Q per k-step. The workspace
//     half-chunks stream through two LDS buffers with direct global->LDS loads
//     (step s + 1 lands while step s is computed; one barrier per step) and serve
//     all four waves; a chunk's logits are formed after its last half. Scores are formed transposed (block j = MFMA row,
//     query = lane column), so the per-row softmax is an in-lane online reduction
//     plus one lane-half exchange; the second pass recomputes the logits, and the
//     per-block sum over the tile's rows is a 16-shuffle transpose-reduction across
//     lanes plus a fixed-order add of the four waves' partial sums.
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

// Sum 16 per-lane registers over the 32 lanes of each lane half; afterwards lane
// col (even) holds the sum of register 8 b4 + 4 b3 + 2 b2 + b1 (bits of col).
__device__ __forceinline__ float transpose_reduce16(float (&v)[16], int col) {
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const bool up = col & 16;
    const float keep = up ? v[i + 8] : v[i];
    const float send = up ? v[i] : v[i + 8];
    v[i] = keep + __shfl_xor(send, 16);
  }
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const bool up = col & 8;
    const float keep = up ? v[i + 4] : v[i];
    const float send = up ? v[i] : v[i + 4];
    v[i] = keep + __shfl_xor(send, 8);
  }
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    const bool up = col & 4;
    const float keep = up ? v[i + 2] : v[i];
    const float send = up ? v[i] : v[i + 2];
    v[i] = keep + __shfl_xor(send, 4);
  }
  {
    const bool up = col & 2;
    const float keep = up ? v[1] : v[0];
    const float send = up ? v[0] : v[1];
    v[0] = keep + __shfl_xor(send, 2);
  }
  return v[0] + __shfl_xor(v[0], 1);
}

// Copy NPART parts (NPART * 8 KB) of one workspace chunk into an LDS buffer with
// direct global->LDS loads: every lane moves 16 bytes per instruction, so one
// instruction of the workgroup moves 4 KB. The consumer waits (vmcnt(0) and a
// barrier) before reading.
template <int NPART>
__device__ __forceinline__ void dma_chunk(const uint16_t* src, uint16_t* lds, int tid) {
  const int w = tid >> 6;
  const uint32_t lds_base =
      (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) uint16_t*)lds;
  const uint32_t voff = (uint32_t)tid * 16u;
#pragma unroll
  for (int i = 0; i < NPART * 2; ++i) {
    const uint32_t m0 =
        __builtin_amdgcn_readfirstlane(lds_base + (uint32_t)(i * kSelThreads + w * 64) * 16u);
    const uint16_t* s = src + i * kSelThreads * 8;
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
// registers; at D = 256 it is formed from Q here (q*q is exact in fp32).
template <bool kSecond, int D, int HF>
__device__ __forceinline__ void selector_products(const uint16_t* ops, int e0,
                                                  const bf16x8 (&qb)[D / 16],
                                                  const bf16x8 (&q2h)[8], const bf16x8 (&q2l)[8],
                                                  f32x16& dmu, f32x16& dvar) {
#pragma unroll
  for (int dc = 0; dc < 8; ++dc) {
    const int off = e0 ^ (dc << 4);
    const bf16x8 q = qb[HF * 8 + dc];
    const bf16x8 mh = as_bf16x8(*reinterpret_cast<const u32x4*>(ops + off));
    const bf16x8 ml = as_bf16x8(*reinterpret_cast<const u32x4*>(ops + kSelPart + off));
    dmu = mfma32(mh, q, dmu);
    dmu = mfma32(ml, q, dmu);
    if (kSecond) {
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
      const bf16x8 vh = as_bf16x8(*reinterpret_cast<const u32x4*>(ops + 2 * kSelPart + off));
      const bf16x8 vl = as_bf16x8(*reinterpret_cast<const u32x4*>(ops + 3 * kSelPart + off));
      dvar = mfma32(vh, sh, dvar);
      dvar = mfma32(vl, sh, dvar);
      dvar = mfma32(vh, sl, dvar);
    }
  }
}

template <int SEL, int D>
__global__ __launch_bounds__(kSelThreads, 2) void selector_kernel(SelArgs a) {
  constexpr bool kSecond = SEL != SPX_SELECTOR_MEAN_BALANCED;
  constexpr bool kDisp = SEL == SPX_SELECTOR_DISPERSION_MEAN;
  constexpr int kParts = kSecond ? 4 : 2;
  constexpr int kHalves = D / 128;
  const int per_tile = a.batch * a.q_heads;
  const int t = a.blocks - 1 - blockIdx.x / per_tile;  // heaviest tiles first
  const int bh = blockIdx.x % per_tile;
  const int b = bh / a.q_heads, h = bh % a.q_heads;
  const int g = h / (a.q_heads / a.kv_heads);
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int col = lane & 31, half = lane >> 5;

  __shared__ __align__(16) uint16_t buf[2][kParts * kSelPart];
  __shared__ float log2_n[kSelMaxBlocks];
  __shared__ float sigma[kDisp ? kSelMaxBlocks : 1];
  __shared__ float part[2][4][kSelChunk];  // by chunk parity: chunk jc is read after
                                           // the next barrier while jc + 1 is written
  __shared__ float tile_score[kSelMaxBlocks];

  const int nchunks = (t + kSelChunk - 1) / kSelChunk;  // visible blocks j < t
  const int pass_steps = nchunks * kHalves;              // (chunk, half) steps per pass
  const uint16_t* src =
      a.ws + ((int64_t)b * a.kv_heads + g) * a.chunks * kHalves * kSelChunkElems;
  if (nchunks > 0) dma_chunk<kParts>(src, buf[0], tid);

  for (int j = tid; j < t; j += kSelThreads) {
    log2_n[j] = log2f((float)a.counts[j]);
    if (kDisp) sigma[j] = a.sigma_v[((int64_t)b * a.blocks + j) * a.kv_heads + g];
  }

  const int64_t qrow = (int64_t)t * kBlock + w * 32 + col;
  const bool row_ok = qrow < a.seq;
  const int tile_rows = min(kBlock, a.seq - t * kBlock);
  bf16x8 qb[D / 16], q2h[8], q2l[8];
  {
    const uint16_t* qsrc = a.q + b * a.qs_b + qrow * a.qs_s + h * a.qs_h + half * 8;
#pragma unroll
    for (int dc = 0; dc < D / 16; ++dc) {
      u32x4 raw = {0u, 0u, 0u, 0u};
      if (row_ok) raw = *reinterpret_cast<const u32x4*>(qsrc + dc * 16);
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

  const float scale_l2 = a.scale * kLog2e;
  const float scale2_half_l2 = 0.5f * a.scale * a.scale * kLog2e;
  const float scale2 = a.scale * a.scale;
  // LDS element offset of this lane's operand row (block col) at 16-byte chunk
  // 2 dc + half: (2 dc + half) ^ (col & 15) = base ^ (dc << 4) in elements.
  const int e0 = col * 128 + (((col >> 1) & 7) << 4) + ((half ^ (col & 1)) << 3);

  float m_run = -INFINITY, l_run = 0.0f;  // per-row softmax state, log2 units
  float inv_l = 0.0f;
  f32x16 dmu = {}, dvar = {};
  const int steps = 2 * pass_steps;
  for (int s = 0; s < steps; ++s) {
    const bool second_pass = s >= pass_steps;
    const int sp = second_pass ? s - pass_steps : s;
    const int jc = sp / kHalves, hf = sp % kHalves;
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    block_sync();  // step s landed everywhere; buffer (s + 1) & 1 is free
    if (second_pass && hf == 0 && jc > 0 && tid < kSelChunk) {
      const int j = (jc - 1) * kSelChunk + tid;
      const float(&pp)[4][kSelChunk] = part[(jc - 1) & 1];
      tile_score[j] = pp[0][tid] + pp[1][tid] + pp[2][tid] + pp[3][tid];
    }
    if (s + 1 < steps) {
      const int ns = s + 1 < pass_steps ? s + 1 : s + 1 - pass_steps;
      dma_chunk<kParts>(src + (int64_t)ns * kSelChunkElems, buf[(s + 1) & 1], tid);
    }
    if (s == pass_steps) {
      // merge the per-row state of the two lane halves (disjoint block sets)
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

    const uint16_t* ops = buf[s & 1];
    if (hf == 0) {
      dmu = f32x16{};
      dvar = f32x16{};
      selector_products<kSecond, D, 0>(ops, e0, qb, q2h, q2l, dmu, dvar);
    } else if constexpr (kHalves > 1) {
      selector_products<kSecond, D, kHalves - 1>(ops, e0, qb, q2h, q2l, dmu, dvar);
    }
    if (hf != kHalves - 1) continue;   // the chunk's other half is still to come

    // logits in log2 units: (scale q.mu + ln n + u / 2) * log2 e; blocks j >= t
    // (only in the last chunk) are masked. Rows past the sequence end (Q = 0) give
    // finite logits and are dropped through inv_l.
    float logit[16];
    const int lim = t - jc * kSelChunk;  // visible rows of this chunk: jr < lim
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int jr = mfma32_row(r, lane);
      const int j = jc * kSelChunk + jr;
      float l2 = fmaf(dmu[r], scale_l2, log2_n[j]);
      if (kSecond) l2 = fmaf(fmaxf(dvar[r], 0.0f), scale2_half_l2, l2);
      logit[r] = l2;
    }
    if (lim < kSelChunk) {
#pragma unroll
      for (int r = 0; r < 16; ++r)
        if (mfma32_row(r, lane) >= lim) logit[r] = -INFINITY;
    }

    if (!second_pass) {
      float mx = -INFINITY;
#pragma unroll
      for (int r = 0; r < 16; ++r) mx = fmaxf(mx, logit[r]);
      const float m_new = fmaxf(m_run, mx);
      if (m_new != -INFINITY) {
        float sum = 0.0f;
#pragma unroll
        for (int r = 0; r < 16; ++r) sum += exp2_fast(logit[r] - m_new);
        l_run = (m_run == -INFINITY ? 0.0f : l_run * exp2_fast(m_run - m_new)) + sum;
        m_run = m_new;
      }
    } else {
      float contrib[16];
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        float p = exp2_fast(logit[r] - m_run) * inv_l;  // m_run finite: t >= 1
        if (kDisp)
          p *= sqrtf(fmaxf(dvar[r], 0.0f) * scale2) * sigma[jc * kSelChunk + mfma32_row(r, lane)];
        contrib[r] = p;
      }
      const float total = transpose_reduce16(contrib, col);
      if ((col & 1) == 0) {
        const int R = 8 * ((col >> 4) & 1) + 4 * ((col >> 3) & 1) + 2 * ((col >> 2) & 1) + ((col >> 1) & 1);
        part[jc & 1][w][mfma32_row(R, lane)] = total;
      }
    }
  }
  block_sync();
  if (nchunks > 0 && tid < kSelChunk) {
    const int j = (nchunks - 1) * kSelChunk + tid;
    const float(&pp)[4][kSelChunk] = part[(nchunks - 1) & 1];
    tile_score[j] = pp[0][tid] + pp[1][tid] + pp[2][tid] + pp[3][tid];
  }
  block_sync();
  const float inv_rows = 1.0f / (float)tile_rows;
  for (int j = tid; j < a.blocks; j += kSelThreads) {
    const float sc = j < t ? tile_score[j] * inv_rows : 0.0f;
    a.score[b * a.ss_b + t * a.ss_t + j * a.ss_j + h * a.ss_h] = sc;
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
  const unsigned grid = (unsigned)(blocks * batch * q_heads);
  if (head_dim == 256) {
    switch (selector) {
      case SPX_SELECTOR_MEAN_BALANCED:
        selector_kernel<SPX_SELECTOR_MEAN_BALANCED, 256><<<grid, kSelThreads, 0, st>>>(a);
        break;
      case SPX_SELECTOR_CGF_MEAN:
        selector_kernel<SPX_SELECTOR_CGF_MEAN, 256><<<grid, kSelThreads, 0, st>>>(a);
        break;
      default:
        selector_kernel<SPX_SELECTOR_DISPERSION_MEAN, 256><<<grid, kSelThreads, 0, st>>>(a);
        break;
    }
  } else {
    switch (selector) {
      case SPX_SELECTOR_MEAN_BALANCED:
        selector_kernel<SPX_SELECTOR_MEAN_BALANCED, 128><<<grid, kSelThreads, 0, st>>>(a);
        break;
      case SPX_SELECTOR_CGF_MEAN:
        selector_kernel<SPX_SELECTOR_CGF_MEAN, 128><<<grid, kSelThreads, 0, st>>>(a);
        break;
      default:
        selector_kernel<SPX_SELECTOR_DISPERSION_MEAN, 128><<<grid, kSelThreads, 0, st>>>(a);
        break;
    }
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
