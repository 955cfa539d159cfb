// Block-sparse causal flash attention (bf16 MFMA, fp32 online softmax in base 2)
// with an optional fused block-mean correction.
//
// Semantics follow upstream/flashprefill_native_forward.py:215-354 (_flash_forward):
// for query tile t and head h, walk the first counts[t, h] entries of the tile's
// index list in order; every listed 128-key block j contributes all its keys
// (keys past the sequence end read as zero), causality is applied only inside the
// block j == t; O = softmax(scale q K^T) V is stored as bf16 and the natural-log
// LSE = M ln 2 + ln l. With the mean correction, each row also attends to the fp32
// block-mean key of every block j < t missing from its list (logit + ln n_j) with
// the block-mean value, inside the same online softmax; this equals the logaddexp
// merge of kernels.py:179-230 (mean_tail) and :312-325 (merge_exact_mean).
//
// gfx950 design
//   * One workgroup (4 waves) per (query tile, q head); wave w owns query rows
//     32w .. 32w + 31 of the tile and keeps them in registers as the B operand.
//   * Scores are computed transposed, S^T = K Q^T, with v_mfma_f32_32x32x16_bf16:
//     each lane owns ONE query column, so the row max / row sum are in-lane
//     reductions plus a single exchange with the other lane half, the O rescale is
//     a per-lane scalar, and the probabilities already sit in the B-operand layout
//     of O^T = V^T P^T: no shuffles and no LDS round trip for P.
//   * K (row-major) and the pre-transposed value tile (from the pooling pass) are
//     staged through LDS with 16-byte accesses; 16-byte chunks are XOR-swizzled by
//     row so the MFMA operand reads are bank-conflict free.
//   * Grid order: (tile, kv group) pairs heaviest-first, and the heads of one
//     group are consecutive on the same XCD (workgroup i runs on XCD i % 8), so the
//     seven q heads sharing a KV block read it from the same L2.
#include "common.h"

namespace spx {

constexpr int kAttnThreads = 256;
constexpr int kMaxBlocksAttn = 1024;
constexpr int kTailTile = 64;  // mean keys per tail tile (hi and lo halves fill K LDS)

struct AttnArgs {
  const uint16_t* q;
  int64_t qs_b, qs_s, qs_h;
  const uint16_t* k;
  int64_t ks_b, ks_s, ks_h;
  const uint16_t* vt;  // [B, Hkv, NB, D, 128]
  const int64_t* idx;  // nullable: all causal blocks
  int64_t is_b, is_t, is_p, is_h;
  const int32_t* cnt;
  int64_t cs_b, cs_t, cs_h;
  const float* mean_k;  // [B, NB, Hkv, D]
  const float* mean_v;
  const int32_t* bcounts;  // [NB]
  void* out;
  int64_t os_b, os_s, os_h;
  float* lse;  // nullable
  int64_t ls_b, ls_s, ls_h;
  int batch, seq, q_heads, kv_heads, blocks, group, num_pairs;
  float scale_log2;
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

// One key tile of the online softmax. s[mb] holds raw q.k dots for key sub-block mb
// (keys 32 mb + mfma32_row(r, lane)) of this lane's query column; only the first
// `nmb` sub-blocks exist. `diag` applies key > query masking inside the tile;
// `bias` (LDS, per key, base-2 units, may be null) is added after scaling.
__device__ __forceinline__ void online_tile(f32x16 (&s)[4], int nmb, bool diag, int qpos,
                                            const float* bias, float scale_log2,
                                            const uint16_t* v_lds, float& m_run,
                                            float& l_run, f32x16 (&o)[4]) {
  const int lane = threadIdx.x & 63;
  const int col = lane & 31, half = lane >> 5;
  float mx = -INFINITY;
#pragma unroll
  for (int mb = 0; mb < 4; ++mb) {
    if (mb < nmb) {
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int key = mb * 32 + mfma32_row(r, lane);
        float x = s[mb][r] * scale_log2;
        if (bias) x += bias[key];
        if (diag && key > qpos) x = -INFINITY;
        s[mb][r] = x;
        mx = fmaxf(mx, x);
      }
    }
  }
  mx = fmaxf(mx, xor32(mx));
  const float m_new = fmaxf(m_run, mx);
  const float corr = (m_run == m_new) ? 1.0f : exp2_fast(m_run - m_new);
  const float msub = (m_new == -INFINITY) ? 0.0f : m_new;
  float rowsum = 0.0f;
  bf16x8 pb[8];
#pragma unroll
  for (int mb = 0; mb < 4; ++mb) {
    if (mb < nmb) {
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const float p = exp2_fast(s[mb][r] - msub);
        s[mb][r] = p;
        rowsum += p;
      }
      pb[2 * mb] = pack8(s[mb], 0);
      pb[2 * mb + 1] = pack8(s[mb], 8);
    }
  }
  l_run = l_run * corr + rowsum;
  m_run = m_new;
  if (corr != 1.0f) {
#pragma unroll
    for (int db = 0; db < 4; ++db) o[db] *= corr;
  }
  // O^T[d][q] += V^T[d][slot] P^T[slot][q]; slot chunk kc covers keys 16 kc .. 16 kc + 15.
#pragma unroll
  for (int kc = 0; kc < 8; ++kc) {
    if (kc < 2 * nmb) {
#pragma unroll
      for (int db = 0; db < 4; ++db) {
        const bf16x8 va = lds_read16(v_lds, swz(db * 32 + col, kc * 2 + half));
        o[db] = mfma32(va, pb[kc], o[db]);
      }
    }
  }
  (void)col;
}

template <bool EXACT, bool TAIL, bool OUT_F32>
__global__ __launch_bounds__(kAttnThreads, 2) void attn_kernel(AttnArgs a) {
  // ---- work item: heaviest (tile, kv group) pairs first, group heads on one XCD
  const int p = blockIdx.x;
  const int xcd = p & 7;
  const int local = p >> 3;
  const int pair_local = local / a.group;
  const int hg = local - pair_local * a.group;
  const int pair = pair_local * 8 + xcd;
  if (pair >= a.num_pairs) return;
  const int bg = a.batch * a.kv_heads;
  const int t = a.blocks - 1 - pair / bg;
  const int b = (pair % bg) / a.kv_heads;
  const int g = (pair % bg) % a.kv_heads;
  const int h = g * a.group + hg;

  __shared__ __align__(16) uint16_t k_lds[kBlock * kBlock];
  __shared__ __align__(16) uint16_t v_lds[kBlock * kBlock];

  const int tid = threadIdx.x;
  const int lane = tid & 63, w = tid >> 6;
  const int col = lane & 31, half = lane >> 5;
  const int qpos = w * 32 + col;  // query position inside the tile
  const int64_t qrow = (int64_t)t * kBlock + qpos;

  bf16x8 qb[8];
  {
    const uint16_t* src = a.q + b * a.qs_b + qrow * a.qs_s + h * a.qs_h + half * 8;
    const bool ok = qrow < a.seq;
#pragma unroll
    for (int dc = 0; dc < 8; ++dc) {
      u32x4 raw = {0u, 0u, 0u, 0u};
      if (ok) raw = *reinterpret_cast<const u32x4*>(src + dc * 16);
      qb[dc] = as_bf16x8(raw);
    }
  }

  float m_run = -INFINITY, l_run = 0.0f;
  f32x16 o[4];
#pragma unroll
  for (int db = 0; db < 4; ++db) o[db] = f32x16{};

  int count;
  if (a.idx) {
    count = a.cnt[b * a.cs_b + t * a.cs_t + h * a.cs_h];
    count = min(max(count, 0), a.blocks);
  } else {
    count = t + 1;
  }
  const int64_t* list = a.idx ? a.idx + b * a.is_b + t * a.is_t + h * a.is_h : nullptr;

  if (EXACT) {
    const uint16_t* kbase = a.k + b * a.ks_b + g * a.ks_h;
    const uint16_t* vbase = a.vt + (((int64_t)b * a.kv_heads + g) * a.blocks) * (kHeadDim * kBlock);
    for (int pos = 0; pos < count; ++pos) {
      const int j = list ? (int)list[pos * a.is_p] : pos;
      if (j < 0 || j >= a.blocks) continue;
      // ---- stage K block j and its value tile into LDS
      u32x4 kr[8], vr[8];
      const uint16_t* vtile = vbase + (int64_t)j * (kHeadDim * kBlock);
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const int id = tid + kAttnThreads * i;
        const int r = id >> 4, c = id & 15;
        const int64_t tok = (int64_t)j * kBlock + r;
        kr[i] = u32x4{0u, 0u, 0u, 0u};
        if (tok < a.seq) kr[i] = *reinterpret_cast<const u32x4*>(kbase + tok * a.ks_s + c * 8);
        vr[i] = *reinterpret_cast<const u32x4*>(vtile + r * kBlock + c * 8);
      }
      __syncthreads();  // previous tile fully consumed
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const int id = tid + kAttnThreads * i;
        const int r = id >> 4, c = id & 15;
        *reinterpret_cast<u32x4*>(k_lds + swz(r, c)) = kr[i];
        *reinterpret_cast<u32x4*>(v_lds + swz(r, c)) = vr[i];
      }
      __syncthreads();

      const bool diag = j == t;
      const int nmb = diag ? (w + 1) : 4;
      f32x16 s[4];
#pragma unroll
      for (int mb = 0; mb < 4; ++mb) s[mb] = f32x16{};
#pragma unroll
      for (int dc = 0; dc < 8; ++dc) {
#pragma unroll
        for (int mb = 0; mb < 4; ++mb) {
          if (mb < nmb) {
            const bf16x8 ka = lds_read16(k_lds, swz(mb * 32 + col, dc * 2 + half));
            s[mb] = mfma32(ka, qb[dc], s[mb]);
          }
        }
      }
      online_tile(s, nmb, diag, qpos, nullptr, a.scale_log2, v_lds, m_run, l_run, o);
    }
  }

  if (TAIL) {
    __shared__ uint32_t listed[kMaxBlocksAttn / 32];
    __shared__ int16_t tail_ids[kMaxBlocksAttn];
    __shared__ float tail_bias[kTailTile];
    __shared__ int wave_counts[4];
    __syncthreads();
    if (tid < kMaxBlocksAttn / 32) listed[tid] = 0u;
    __syncthreads();
    for (int pos = tid; pos < count; pos += kAttnThreads) {
      const int j = list ? (int)list[pos * a.is_p] : pos;
      if (j >= 0 && j < a.blocks) atomicOr(&listed[j >> 5], 1u << (j & 31));
    }
    __syncthreads();
    // ascending compaction of {j < t : j not listed}
    int ntail = 0;
    for (int j0 = 0; j0 < t; j0 += kAttnThreads) {
      const int j = j0 + tid;
      const bool in_tail = j < t && ((listed[j >> 5] >> (j & 31)) & 1u) == 0u;
      const uint64_t ballot = __ballot(in_tail);
      const int before = __popcll(ballot & ((1ull << lane) - 1ull));
      if (lane == 0) wave_counts[w] = __popcll(ballot);
      __syncthreads();
      int offset = ntail;
      for (int x = 0; x < w; ++x) offset += wave_counts[x];
      if (in_tail) tail_ids[offset + before] = (int16_t)j;
      for (int x = 0; x < 4; ++x) ntail += wave_counts[x];
      __syncthreads();
    }

    const int64_t desc_base = (int64_t)b * a.blocks * a.kv_heads + g;  // (b, 0, g) row
    for (int t0 = 0; t0 < ntail; t0 += kTailTile) {
      __syncthreads();
      // stage: K rows i (hi) and 64 + i (lo) of mean K; value slots 0..63 of mean V
      for (int e = tid; e < kTailTile * kHeadDim; e += kAttnThreads) {
        const int i = e >> 7, d = e & 127;
        const int j = (t0 + i < ntail) ? (int)tail_ids[t0 + i] : -1;
        float mk = 0.0f, mv = 0.0f;
        if (j >= 0) {
          const int64_t off = (desc_base + (int64_t)j * a.kv_heads) * kHeadDim + d;
          mk = a.mean_k[off];
          mv = a.mean_v[off];
        }
        const uint16_t hi = to_bf16_bits(mk);
        const uint16_t lo = to_bf16_bits(mk - __uint_as_float((uint32_t)hi << 16));
        k_lds[swz(i, d >> 3) + (d & 7)] = hi;
        k_lds[swz(kTailTile + i, d >> 3) + (d & 7)] = lo;
        const int slot = value_slot_of_key(i);
        v_lds[swz(d, slot >> 3) + (slot & 7)] = to_bf16_bits(mv);
        if (d == 0)
          tail_bias[i] = j >= 0 ? __logf((float)a.bcounts[j]) * kLog2e : -INFINITY;
      }
      __syncthreads();
      f32x16 s[4];
#pragma unroll
      for (int mb = 0; mb < 4; ++mb) s[mb] = f32x16{};
#pragma unroll
      for (int dc = 0; dc < 8; ++dc) {
#pragma unroll
        for (int mb = 0; mb < 2; ++mb) {
          const bf16x8 khi = lds_read16(k_lds, swz(mb * 32 + col, dc * 2 + half));
          const bf16x8 klo = lds_read16(k_lds, swz(kTailTile + mb * 32 + col, dc * 2 + half));
          s[mb] = mfma32(khi, qb[dc], s[mb]);
          s[mb] = mfma32(klo, qb[dc], s[mb]);
        }
      }
      online_tile(s, 2, false, qpos, tail_bias, a.scale_log2, v_lds, m_run, l_run, o);
    }
  }

  // ---- epilogue
  const float l = l_run + xor32(l_run);
  const bool any = l > 0.0f;
  const float inv = any ? 1.0f / l : 0.0f;
  if (qrow < a.seq) {
    if (OUT_F32) {
      float* dst = static_cast<float*>(a.out) + b * a.os_b + qrow * a.os_s + h * a.os_h;
#pragma unroll
      for (int db = 0; db < 4; ++db) {
#pragma unroll
        for (int rr = 0; rr < 4; ++rr) {
          const int d0 = db * 32 + 8 * rr + 4 * half;
          f32x4 v4 = {o[db][4 * rr] * inv, o[db][4 * rr + 1] * inv, o[db][4 * rr + 2] * inv,
                      o[db][4 * rr + 3] * inv};
          *reinterpret_cast<f32x4*>(dst + d0) = v4;
        }
      }
    } else {
      uint16_t* dst = static_cast<uint16_t*>(a.out) + b * a.os_b + qrow * a.os_s + h * a.os_h;
#pragma unroll
      for (int db = 0; db < 4; ++db) {
#pragma unroll
        for (int rr = 0; rr < 4; ++rr) {
          const int d0 = db * 32 + 8 * rr + 4 * half;
          u32x2 v2;
          v2[0] = pack_bf16x2(o[db][4 * rr] * inv, o[db][4 * rr + 1] * inv);
          v2[1] = pack_bf16x2(o[db][4 * rr + 2] * inv, o[db][4 * rr + 3] * inv);
          *reinterpret_cast<u32x2*>(dst + d0) = v2;
        }
      }
    }
    if (a.lse && half == 0)
      a.lse[b * a.ls_b + qrow * a.ls_s + h * a.ls_h] = any ? m_run * kLn2 + __logf(l) : -INFINITY;
  }
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
  int batch, seq, heads;
};

// One wave per (b, s, h) row of 128 dims; each lane handles 2 dims.
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
  const int d = lane * 2;
  const uint32_t e2 = *reinterpret_cast<const uint32_t*>(a.eo + b * a.es_b + s * a.es_s + h * a.es_h + d);
  const float* m2 = a.mo + b * a.ms_b + s * a.ms_s + h * a.ms_h + d;
  const float o0 = bf16_lo(e2) * we + m2[0] * wm;
  const float o1 = bf16_hi(e2) * we + m2[1] * wm;
  *reinterpret_cast<uint32_t*>(a.out + b * a.os_b + s * a.os_s + h * a.os_h + d) = pack_bf16x2(o0, o1);
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
};

int launch_attention(const AttnRequest& req, const void* q, const int64_t* q_strides,
                     const void* k, const int64_t* k_strides, const void* value_tiles,
                     const int64_t* indices, const int64_t* index_strides,
                     const int32_t* counts, const int64_t* count_strides,
                     const float* mean_k, const float* mean_v, const int32_t* block_counts,
                     int batch, int seq, int q_heads, int kv_heads, int head_dim,
                     int block_size, float scale, void* out, const int64_t* out_strides,
                     float* lse, const int64_t* lse_strides, void* stream) {
  SPX_REQUIRE(head_dim == kHeadDim, SPX_EUNSUPPORTED, "head_dim %d unsupported (only 128)", head_dim);
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
    e = check_bsdh("k", k, k_strides, true);
    if (e) return e;
    SPX_REQUIRE(value_tiles != nullptr && (reinterpret_cast<uintptr_t>(value_tiles) & 15) == 0,
                SPX_EINVAL, "value_tiles: null or not 16-byte aligned");
  }
  if (req.tail) {
    SPX_REQUIRE(mean_k && mean_v && block_counts, SPX_EINVAL,
                "mean correction needs mean_k, mean_v and block_counts");
  }
  if (indices) {
    SPX_REQUIRE(index_strides && counts && count_strides, SPX_EINVAL,
                "indices given without strides / counts");
  } else {
    SPX_REQUIRE(req.exact, SPX_EINVAL, "mean_tail needs index lists");
  }
  if (lse) SPX_REQUIRE(lse_strides != nullptr, SPX_EINVAL, "lse strides missing");

  AttnArgs a{};
  a.q = static_cast<const uint16_t*>(q);
  a.qs_b = q_strides[0]; a.qs_s = q_strides[1]; a.qs_h = q_strides[2];
  a.k = static_cast<const uint16_t*>(k);
  if (req.exact) { a.ks_b = k_strides[0]; a.ks_s = k_strides[1]; a.ks_h = k_strides[2]; }
  a.vt = static_cast<const uint16_t*>(value_tiles);
  a.idx = indices;
  if (indices) {
    a.is_b = index_strides[0]; a.is_t = index_strides[1]; a.is_p = index_strides[2];
    a.is_h = index_strides[3];
    a.cnt = counts;
    a.cs_b = count_strides[0]; a.cs_t = count_strides[1]; a.cs_h = count_strides[2];
  }
  a.mean_k = mean_k; a.mean_v = mean_v; a.bcounts = block_counts;
  a.out = out;
  a.os_b = out_strides[0]; a.os_s = out_strides[1]; a.os_h = out_strides[2];
  a.lse = lse;
  if (lse) { a.ls_b = lse_strides[0]; a.ls_s = lse_strides[1]; a.ls_h = lse_strides[2]; }
  a.batch = batch; a.seq = seq; a.q_heads = q_heads; a.kv_heads = kv_heads;
  a.blocks = blocks; a.group = q_heads / kv_heads;
  a.num_pairs = blocks * batch * kv_heads;
  a.scale_log2 = (float)((double)scale * 1.4426950408889634);
  const int grid = ((a.num_pairs + 7) / 8) * 8 * a.group;
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (req.exact && !req.tail) attn_kernel<true, false, false><<<grid, kAttnThreads, 0, st>>>(a);
  else if (req.exact && req.tail) attn_kernel<true, true, false><<<grid, kAttnThreads, 0, st>>>(a);
  else attn_kernel<false, true, true><<<grid, kAttnThreads, 0, st>>>(a);
  return launch_status("attention");
}

}  // namespace

extern "C" int spx_exact_attention(const void* q, const int64_t* q_strides, const void* k,
                                   const int64_t* k_strides, const void* value_tiles,
                                   const int64_t* indices, const int64_t* index_strides,
                                   const int32_t* counts, const int64_t* count_strides, int batch,
                                   int seq, int q_heads, int kv_heads, int head_dim,
                                   int block_size, float scale, void* out,
                                   const int64_t* out_strides, float* lse,
                                   const int64_t* lse_strides, void* stream) {
  return launch_attention({true, false, false}, q, q_strides, k, k_strides, value_tiles, indices,
                          index_strides, counts, count_strides, nullptr, nullptr, nullptr, batch,
                          seq, q_heads, kv_heads, head_dim, block_size, scale, out, out_strides,
                          lse, lse_strides, stream);
}

extern "C" int spx_sparse_attention_mean(const void* q, const int64_t* q_strides, const void* k,
                                         const int64_t* k_strides, const void* value_tiles,
                                         const int64_t* indices, const int64_t* index_strides,
                                         const int32_t* counts, const int64_t* count_strides,
                                         const float* mean_k, const float* mean_v,
                                         const int32_t* block_counts, int batch, int seq,
                                         int q_heads, int kv_heads, int head_dim, int block_size,
                                         float scale, void* out, const int64_t* out_strides,
                                         float* lse, const int64_t* lse_strides, void* stream) {
  return launch_attention({true, true, false}, q, q_strides, k, k_strides, value_tiles, indices,
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
  return launch_attention({false, true, true}, q, q_strides, nullptr, nullptr, nullptr, indices,
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
  SPX_REQUIRE(head_dim == kHeadDim, SPX_EUNSUPPORTED, "head_dim %d unsupported (only 128)", head_dim);
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
  a.batch = batch; a.seq = seq; a.heads = heads;
  const int64_t rows = (int64_t)batch * seq * heads;
  const int grid = (int)((rows + 3) / 4);
  merge_kernel<<<grid, 256, 0, static_cast<hipStream_t>(stream)>>>(a);
  return launch_status("merge_exact_mean");
}
