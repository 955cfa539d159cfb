// Shared device helpers for the gfx950 sparse-prefill kernels.
//
// Everything here is CDNA4-specific: 64-lane wavefronts, bf16 MFMA through
// __builtin_amdgcn_mfma_f32_32x32x16_bf16, hardware v_exp_f32 and
// v_cvt_pk_bf16_f32. There is no other code path.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "sparse_prefill.h"

namespace spx {

constexpr int kWave = 64;
constexpr int kBlock = 128;      // routing block and query tile (tokens)
constexpr int kHeadDim = 128;    // Qwen2.5-7B head_dim
constexpr float kLog2e = 1.4426950408889634f;
constexpr float kLn2 = 0.6931471805599453f;

typedef __bf16 bf16;
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

// ---------------------------------------------------------------- bf16 bits

__device__ __forceinline__ float bf16_lo(uint32_t w) { return __uint_as_float(w << 16); }
__device__ __forceinline__ float bf16_hi(uint32_t w) { return __uint_as_float(w & 0xffff0000u); }

// Round-to-nearest-even float -> bf16 (v_cvt_pk_bf16_f32 on gfx950).
__device__ __forceinline__ uint32_t pack_bf16x2(float a, float b) {
  typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
  bf16x2 p;
  p[0] = (__bf16)a;
  p[1] = (__bf16)b;
  return __builtin_bit_cast(uint32_t, p);
}

__device__ __forceinline__ uint16_t to_bf16_bits(float a) {
  return (uint16_t)(pack_bf16x2(a, 0.0f) & 0xffffu);
}

__device__ __forceinline__ float exp2_fast(float x) { return __builtin_amdgcn_exp2f(x); }

// NaN-propagating max (torch.amax semantics).
__device__ __forceinline__ float max_nan(float a, float b) {
  if (a != a) return a;
  if (b != b) return b;
  return a > b ? a : b;
}

// ------------------------------------------------------------------- MFMA
//
// v_mfma_f32_32x32x16_bf16: D[32x32] += A[32x16] * B[16x32].
//   A operand: lane l holds A[l % 32][8 * (l / 32) + 0..7]
//   B operand: lane l holds B[8 * (l / 32) + 0..7][l % 32]
//   C/D:       lane l, register r holds D[8 * (r / 4) + 4 * (l / 32) + r % 4][l % 32]
__device__ __forceinline__ f32x16 mfma32(const bf16x8& a, const bf16x8& b, const f32x16& c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
}

__device__ __forceinline__ int mfma32_row(int r, int lane) {
  return 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
}

__device__ __forceinline__ bf16x8 as_bf16x8(const u32x4& v) {
  return __builtin_bit_cast(bf16x8, v);
}

// ------------------------------------------------------------ lane shuffles

__device__ __forceinline__ float xor32(float v) { return __shfl_xor(v, 32); }

// Keep `x` opaque inside a loop so values derived from it are recomputed per use
// instead of being hoisted (and held in registers) as loop invariants.
__device__ __forceinline__ int opaque(int x) {
  asm volatile("" : "+v"(x));
  return x;
}

// Eight consecutive fp32 values (16-byte aligned) as two 16-byte loads.
__device__ __forceinline__ void load8(const float* p, float (&x)[8]) {
  const f32x4 a0 = *reinterpret_cast<const f32x4*>(p);
  const f32x4 a1 = *reinterpret_cast<const f32x4*>(p + 4);
#pragma unroll
  for (int e = 0; e < 4; ++e) { x[e] = a0[e]; x[4 + e] = a1[e]; }
}

__device__ __forceinline__ float wave_max(float v) {
  for (int o = 32; o >= 1; o >>= 1) v = max_nan(v, __shfl_xor(v, o));
  return v;
}

__device__ __forceinline__ float wave_sum(float v) {
  for (int o = 32; o >= 1; o >>= 1) v += __shfl_xor(v, o);
  return v;
}

// Workgroup barrier preceded by an explicit wait for this wave's outstanding LDS
// operations. __syncthreads() alone is not enough: at a loop-header barrier whose
// back edge carries an LDS store, hipcc has emitted s_barrier with the store still
// in flight, and another wave then read the old value right after the barrier.
// Every kernel here synchronises through this helper.
__device__ __forceinline__ void block_sync() {
  asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
  __syncthreads();
}

// --------------------------------------------------------------- geometry

__host__ __device__ __forceinline__ int num_blocks(int seq) { return (seq + kBlock - 1) / kBlock; }

// Value tiles: V of each (batch, kv head, key block) stored transposed as
// [dim][128 key slots] bf16. Inside every 16-key chunk the keys are permuted so
// that the 8 keys one MFMA lane-half consumes are contiguous:
//   slot s (0..15) holds key 4 * (s / 8) + (s % 4) + 8 * ((s % 8) / 4).
__host__ __device__ __forceinline__ int value_slot_of_key(int key) {
  const int chunk = key >> 4, kk = key & 15;
  const int half = (kk >> 2) & 1;
  const int m = (kk & 3) + 4 * (kk >> 3);
  return chunk * 16 + half * 8 + m;
}

}  // namespace spx

// ------------------------------------------------------------ host errors

namespace spx {
void set_error(const char* fmt, ...);
int launch_status(const char* what);
// What a d = 256 attention launch computes besides / instead of the exact blocks
// (the tails mirror the d = 128 kernel's: block means, or rescue tokens with an
// optional remainder entry), and whether the output is fp32.
struct Attn256Options {
  bool exact, tail, out_f32;
  int tail_kind;               // 0 block means, 1 rescue token, 2 rescue token + remainder
  const float* mean_k;         // [B, NB, Hkv, 256] fp32 (tail_kind 0 and 2)
  const float* mean_v;
  const int32_t* block_counts; // [NB] (tail_kind 0)
  const uint8_t* choice;       // [B, NB, NB, Hq] rescue token per (tile, block, head)
  const void* v;               // V rows of the rescue tokens, strided [B, S, Hkv, 256]
  const int64_t* v_strides;
  int32_t* work_queue;         // optional zeroed counter: the last third of the tiles dealt dynamically
};
// Attention at head_dim 256 (attn256.hip); arguments as spx_exact_attention and the
// tail entry points, already validated by the caller.
int launch_attention_256(const Attn256Options& opt, const void* q, const int64_t* q_strides,
                         const void* key_tiles, const void* value_tiles, const int64_t* indices,
                         const int64_t* index_strides, const int32_t* counts,
                         const int64_t* count_strides, int batch, int seq, int q_heads,
                         int kv_heads, float scale, void* out, const int64_t* out_strides,
                         float* lse, const int64_t* lse_strides, void* stream);
}  // namespace spx

#define SPX_REQUIRE(cond, code, ...)        \
  do {                                      \
    if (!(cond)) {                          \
      ::spx::set_error(__VA_ARGS__);        \
      return (code);                        \
    }                                       \
  } while (0)
