// C-ABI plumbing (thread-local error text, launch status) and the integer
// selection-accounting counters of kernels.py:328-407.
#include <stdarg.h>
#include <stdio.h>

#include "common.h"

namespace spx {

static thread_local char g_error[512] = "";

void set_error(const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_error, sizeof(g_error), fmt, ap);
  va_end(ap);
}

int launch_status(const char* what) {
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) {
    set_error("%s: launch failed: %s", what, hipGetErrorString(e));
    return SPX_ELAUNCH;
  }
  return SPX_OK;
}

__global__ void zero_i64_kernel(int64_t* p, int n) {
  if ((int)threadIdx.x < n) p[threadIdx.x] = 0;
}

// One workgroup per (batch, query block t); threads stride over (key block, head).
__global__ __launch_bounds__(256) void accounting_kernel(const uint8_t* mask, int blocks, int heads,
                                                         int seq, int q_tile, int64_t* totals) {
  const int t = blockIdx.x % blocks;
  const int b = blockIdx.x / blocks;
  const int64_t nt = min(kBlock, seq - t * kBlock);
  const int64_t row = ((int64_t)b * blocks + t) * blocks * heads;
  int64_t pairs = 0, selected = 0, tail = 0;
  for (int e = threadIdx.x; e < blocks * heads; e += blockDim.x) {
    const int j = e / heads;
    const bool sel = mask[row + e] != 0;
    if (sel) {
      ++selected;
      if (j < t) pairs += nt * (int64_t)min(kBlock, seq - j * kBlock);
      else if (j == t) pairs += nt * (nt + 1) / 2;
    } else if (j < t) {
      tail += nt;
    }
  }
  __shared__ int64_t red[3][256];
  red[0][threadIdx.x] = pairs;
  red[1][threadIdx.x] = selected;
  red[2][threadIdx.x] = tail;
  block_sync();
  for (int s = 128; s > 0; s >>= 1) {
    if ((int)threadIdx.x < s) {
      red[0][threadIdx.x] += red[0][threadIdx.x + s];
      red[1][threadIdx.x] += red[1][threadIdx.x + s];
      red[2][threadIdx.x] += red[2][threadIdx.x + s];
    }
    block_sync();
  }
  if (threadIdx.x == 0) {
    atomicAdd(reinterpret_cast<unsigned long long*>(&totals[0]), (unsigned long long)red[0][0]);
    atomicAdd(reinterpret_cast<unsigned long long*>(&totals[1]), (unsigned long long)red[1][0]);
    atomicAdd(reinterpret_cast<unsigned long long*>(&totals[2]), (unsigned long long)red[2][0]);
    if (q_tile > 0) {
      const int64_t programs = (nt + q_tile - 1) / q_tile;
      atomicAdd(reinterpret_cast<unsigned long long*>(&totals[3]),
                (unsigned long long)(red[1][0] * programs));
    }
  }
}

}  // namespace spx

using namespace spx;

extern "C" const char* spx_last_error(void) { return g_error; }

extern "C" int spx_abi_version(void) { return SPX_ABI_VERSION; }

extern "C" int spx_selection_accounting(const uint8_t* mask, int batch, int blocks, int heads,
                                        int seq, int block_size, int q_tile, int64_t* totals,
                                        void* stream) {
  SPX_REQUIRE(mask && totals, SPX_EINVAL, "null pointer");
  SPX_REQUIRE(block_size == kBlock, SPX_EUNSUPPORTED, "block_size %d unsupported (only 128)",
              block_size);
  SPX_REQUIRE(batch > 0 && heads > 0 && seq > 0 && blocks == num_blocks(seq), SPX_EINVAL,
              "bad accounting shape: batch %d blocks %d heads %d seq %d", batch, blocks, heads, seq);
  hipStream_t st = static_cast<hipStream_t>(stream);
  zero_i64_kernel<<<1, 64, 0, st>>>(totals, 4);
  accounting_kernel<<<batch * blocks, 256, 0, st>>>(mask, blocks, heads, seq, q_tile, totals);
  return launch_status("selection_accounting");
}
