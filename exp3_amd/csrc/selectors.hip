// Balanced / CGF / dispersion block scores (kernels.py:49-126).
//
// For each real row r of tile t, head h and visible block j < t:
//   l0 = scale * q.mu_K,j + ln n_j
//   u  = max(0, scale^2 * (q*q).var_K,j)
//   logit = l0 (mean_balanced) | l0 + u / 2 (cgf_mean, dispersion_mean)
//   p = softmax over j < t ; contribution = p | p * sqrt(u) * sigma_V,j (dispersion)
//   score[t, j] = mean over the tile's real rows (0 for j >= t and for t = 0).
//
// gfx950 mapping: one workgroup per (tile, q head), four waves of 32 query rows.
// The two dot products are MFMA GEMMs against the fp32 descriptors, kept to about
// fp32 accuracy by splitting every fp32 operand into bf16 hi + lo parts
// (q is bf16-exact; q*q is exact in fp32 and splits exactly into two bf16):
//   q.mu  = q.mu_hi + q.mu_lo                      (2 MFMA)
//   q2.var = q2_hi.var_hi + q2_hi.var_lo + q2_lo.var_hi   (3 MFMA, drops 2^-16 term)
// Scores are formed transposed (block j = MFMA row, query = lane column), so the
// per-row softmax is an in-lane online reduction plus one lane-half exchange; a
// second pass recomputes the logits, and the per-block sum over the tile's rows
// is a 16-shuffle transpose-reduction across lanes plus an LDS add across waves.
#include "common.h"

namespace spx {

constexpr int kSelThreads = 256;
constexpr int kSelMaxBlocks = 1024;

struct SelArgs {
  const uint16_t* q;
  int64_t qs_b, qs_s, qs_h;
  const float* mean_k;   // [B, NB, Hkv, D]
  const float* var_k;
  const float* sigma_v;  // [B, NB, Hkv]
  const int32_t* counts; // [NB]
  int batch, seq, q_heads, kv_heads, blocks;
  int selector;
  float scale;
  float* score;
  int64_t ss_b, ss_t, ss_j, ss_h;
};

__device__ __forceinline__ int sswz(int row, int chunk) {
  return row * kHeadDim + ((chunk ^ (row & 15)) << 3);
}

__device__ __forceinline__ void split8(const float* v, u32x4& hi, u32x4& lo) {
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    const uint32_t h2 = pack_bf16x2(v[2 * e], v[2 * e + 1]);
    hi[e] = h2;
    lo[e] = pack_bf16x2(v[2 * e] - bf16_lo(h2), v[2 * e + 1] - bf16_hi(h2));
  }
}

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

__global__ __launch_bounds__(kSelThreads) void selector_kernel(SelArgs a) {
  const int per_tile = a.batch * a.q_heads;
  const int t = a.blocks - 1 - blockIdx.x / per_tile;
  const int bh = blockIdx.x % per_tile;
  const int b = bh / a.q_heads, h = bh % a.q_heads;
  const int g = h / (a.q_heads / a.kv_heads);
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int col = lane & 31, half = lane >> 5;
  const bool second_order = a.selector != SPX_SELECTOR_MEAN_BALANCED;
  const bool dispersion = a.selector == SPX_SELECTOR_DISPERSION_MEAN;

  __shared__ __align__(16) uint16_t mu_hi[32 * kHeadDim];
  __shared__ __align__(16) uint16_t mu_lo[32 * kHeadDim];
  __shared__ __align__(16) uint16_t var_hi[32 * kHeadDim];
  __shared__ __align__(16) uint16_t var_lo[32 * kHeadDim];
  __shared__ float blk_log_n[32];
  __shared__ float blk_sigma[32];
  __shared__ float part[4][kSelMaxBlocks];  // per-wave row sums, added in fixed order

  const int64_t qrow = (int64_t)t * kBlock + w * 32 + col;
  const bool row_ok = qrow < a.seq;
  const int tile_rows = min(kBlock, a.seq - t * kBlock);
  bf16x8 qb[8], q2h[8], q2l[8];
  {
    const uint16_t* src = a.q + b * a.qs_b + qrow * a.qs_s + h * a.qs_h + half * 8;
#pragma unroll
    for (int dc = 0; dc < 8; ++dc) {
      u32x4 raw = {0u, 0u, 0u, 0u};
      if (row_ok) raw = *reinterpret_cast<const u32x4*>(src + dc * 16);
      qb[dc] = as_bf16x8(raw);
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

  const int nchunks = (t + 31) / 32;  // visible blocks j < t
  const float scale2 = a.scale * a.scale;
  const int64_t dbase = (int64_t)b * a.blocks * a.kv_heads + g;

  float m_run = -INFINITY, l_run = 0.0f;  // per-row softmax state (this lane's blocks)

  for (int pass = 0; pass < 2; ++pass) {
    for (int jc = 0; jc < nchunks; ++jc) {
      __syncthreads();
      for (int e = tid; e < 32 * 16; e += kSelThreads) {
        const int r = e >> 4, c = e & 15;
        const int j = jc * 32 + r;
        float mu[8] = {}, var[8] = {};
        if (j < t) {
          const int64_t off = (dbase + (int64_t)j * a.kv_heads) * kHeadDim + c * 8;
          const f32x4* pm = reinterpret_cast<const f32x4*>(a.mean_k + off);
          const f32x4 m0 = pm[0], m1 = pm[1];
#pragma unroll
          for (int x = 0; x < 4; ++x) { mu[x] = m0[x]; mu[4 + x] = m1[x]; }
          if (second_order) {
            const f32x4* pv = reinterpret_cast<const f32x4*>(a.var_k + off);
            const f32x4 v0 = pv[0], v1 = pv[1];
#pragma unroll
            for (int x = 0; x < 4; ++x) { var[x] = v0[x]; var[4 + x] = v1[x]; }
          }
        }
        u32x4 hi, lo;
        split8(mu, hi, lo);
        *reinterpret_cast<u32x4*>(mu_hi + sswz(r, c)) = hi;
        *reinterpret_cast<u32x4*>(mu_lo + sswz(r, c)) = lo;
        if (second_order) {
          split8(var, hi, lo);
          *reinterpret_cast<u32x4*>(var_hi + sswz(r, c)) = hi;
          *reinterpret_cast<u32x4*>(var_lo + sswz(r, c)) = lo;
        }
        if (c == 0) {
          blk_log_n[r] = j < t ? logf((float)a.counts[j]) : 0.0f;
          blk_sigma[r] = (dispersion && j < t) ? a.sigma_v[dbase + (int64_t)j * a.kv_heads] : 0.0f;
        }
      }
      __syncthreads();

      f32x16 dmu = {}, dvar = {};
#pragma unroll
      for (int dc = 0; dc < 8; ++dc) {
        const int off = sswz(col, dc * 2 + half);
        dmu = mfma32(as_bf16x8(*reinterpret_cast<const u32x4*>(mu_hi + off)), qb[dc], dmu);
        dmu = mfma32(as_bf16x8(*reinterpret_cast<const u32x4*>(mu_lo + off)), qb[dc], dmu);
        if (second_order) {
          const bf16x8 vh = as_bf16x8(*reinterpret_cast<const u32x4*>(var_hi + off));
          const bf16x8 vl = as_bf16x8(*reinterpret_cast<const u32x4*>(var_lo + off));
          dvar = mfma32(vh, q2h[dc], dvar);
          dvar = mfma32(vl, q2h[dc], dvar);
          dvar = mfma32(vh, q2l[dc], dvar);
        }
      }

      float logit[16], mult[16];
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int jr = mfma32_row(r, lane);
        const int j = jc * 32 + jr;
        const bool visible = j < t && row_ok;
        float l0 = dmu[r] * a.scale + blk_log_n[jr];
        float m = 1.0f;
        if (second_order) {
          const float u = fmaxf(dvar[r] * scale2, 0.0f);
          l0 += 0.5f * u;
          if (dispersion) m = sqrtf(u) * blk_sigma[jr];
        }
        logit[r] = visible ? l0 : -INFINITY;
        mult[r] = m;
      }

      if (pass == 0) {
        float mx = -INFINITY;
#pragma unroll
        for (int r = 0; r < 16; ++r) mx = fmaxf(mx, logit[r]);
        const float m_new = fmaxf(m_run, mx);
        if (m_new != -INFINITY) {
          float s = 0.0f;
#pragma unroll
          for (int r = 0; r < 16; ++r) s += exp2_fast((logit[r] - m_new) * kLog2e);
          l_run = (m_run == -INFINITY ? 0.0f : l_run * exp2_fast((m_run - m_new) * kLog2e)) + s;
          m_run = m_new;
        }
      } else {
        float contrib[16];
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const float p = logit[r] == -INFINITY ? 0.0f : exp2_fast((logit[r] - m_run) * kLog2e) / l_run;
          contrib[r] = p * mult[r];
        }
        const float total = transpose_reduce16(contrib, col);
        if ((col & 1) == 0) {
          const int R = 8 * ((col >> 4) & 1) + 4 * ((col >> 3) & 1) + 2 * ((col >> 2) & 1) + ((col >> 1) & 1);
          const int j = jc * 32 + mfma32_row(R, lane);
          if (j < t) part[w][j] = total;
        }
      }
    }
    if (pass == 0) {
      // merge the per-row state of the two lane halves (disjoint block sets)
      const float om = xor32(m_run), ol = xor32(l_run);
      const float nm = fmaxf(m_run, om);
      if (nm != -INFINITY) {
        l_run = (m_run == -INFINITY ? 0.0f : l_run * exp2_fast((m_run - nm) * kLog2e)) +
                (om == -INFINITY ? 0.0f : ol * exp2_fast((om - nm) * kLog2e));
      }
      m_run = nm;
    }
  }
  __syncthreads();
  const float inv_rows = 1.0f / (float)tile_rows;
  for (int j = tid; j < a.blocks; j += kSelThreads) {
    const float s = j < t ? (part[0][j] + part[1][j] + part[2][j] + part[3][j]) * inv_rows : 0.0f;
    a.score[b * a.ss_b + t * a.ss_t + j * a.ss_j + h * a.ss_h] = s;
  }
}

}  // namespace spx

using namespace spx;

extern "C" int spx_selector_scores(const void* q, const int64_t* q_strides, const float* mean_k,
                                   const float* var_k, const float* sigma_v, const int32_t* counts,
                                   int batch, int seq, int q_heads, int kv_heads, int head_dim,
                                   int block_size, int selector, float scale, float* score,
                                   const int64_t* score_strides, void* stream) {
  SPX_REQUIRE(selector == SPX_SELECTOR_MEAN_BALANCED || selector == SPX_SELECTOR_CGF_MEAN ||
                  selector == SPX_SELECTOR_DISPERSION_MEAN,
              SPX_EINVAL, "unsupported selector id %d", selector);
  SPX_REQUIRE(head_dim == kHeadDim, SPX_EUNSUPPORTED, "head_dim %d unsupported (only 128)", head_dim);
  SPX_REQUIRE(block_size == kBlock, SPX_EUNSUPPORTED, "block_size %d unsupported (only 128)", block_size);
  SPX_REQUIRE(batch > 0 && seq > 0 && q_heads > 0 && kv_heads > 0 && q_heads % kv_heads == 0,
              SPX_EINVAL, "bad shape");
  SPX_REQUIRE(q && q_strides && q_strides[3] == 1 && (reinterpret_cast<uintptr_t>(q) & 15) == 0 &&
                  q_strides[0] % 8 == 0 && q_strides[1] % 8 == 0 && q_strides[2] % 8 == 0,
              SPX_EINVAL, "q: null, misaligned or non-unit dim stride");
  SPX_REQUIRE(mean_k && counts && score && score_strides, SPX_EINVAL, "null pointer");
  SPX_REQUIRE((reinterpret_cast<uintptr_t>(mean_k) & 15) == 0 &&
                  (reinterpret_cast<uintptr_t>(var_k) & 15) == 0,
              SPX_EINVAL, "mean_k / var_k must be 16-byte aligned");
  SPX_REQUIRE(selector == SPX_SELECTOR_MEAN_BALANCED || var_k, SPX_EINVAL, "var_k: null pointer");
  SPX_REQUIRE(selector != SPX_SELECTOR_DISPERSION_MEAN || sigma_v, SPX_EINVAL, "sigma_v: null pointer");
  const int blocks = num_blocks(seq);
  SPX_REQUIRE(blocks <= kSelMaxBlocks, SPX_EUNSUPPORTED, "seq %d exceeds %d blocks", seq, kSelMaxBlocks);
  SelArgs a{};
  a.q = static_cast<const uint16_t*>(q);
  a.qs_b = q_strides[0]; a.qs_s = q_strides[1]; a.qs_h = q_strides[2];
  a.mean_k = mean_k; a.var_k = var_k; a.sigma_v = sigma_v; a.counts = counts;
  a.batch = batch; a.seq = seq; a.q_heads = q_heads; a.kv_heads = kv_heads; a.blocks = blocks;
  a.selector = selector;
  a.scale = scale;
  a.score = score;
  a.ss_b = score_strides[0]; a.ss_t = score_strides[1]; a.ss_j = score_strides[2];
  a.ss_h = score_strides[3];
  selector_kernel<<<blocks * batch * q_heads, kSelThreads, 0, static_cast<hipStream_t>(stream)>>>(a);
  return launch_status("selector_scores");
}
