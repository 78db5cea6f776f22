// K0 (NF4 blockwise quantise) and K1 (standalone NF4 -> bf16 dequant) for gfx950.
//
// K0 moves 2 B in and 0.5625 B out per value; with blocksize 64 (the expert path) eight
// lanes share a block and every wave reads and writes contiguous runs.
//
// K1 is HBM-bound: 0.5 B read + 2 B written per value (plus 4 B of absmax per 64
// values).  Each thread owns 32 consecutive values: one 16-byte load of packed nibbles,
// one absmax, four 16-byte stores of bf16.  The 16-entry codebook sits in LDS; 16
// distinct entries map to 16 distinct banks, so the lookups never conflict.
#include "common.h"

namespace moe {
namespace {

constexpr int kDequantThreads = 256;
// A wave dequantises chunks of 2048 values: lane l handles the 8 values at 512*s + 8*l of
// each quarter s, so each of its four 16-byte stores is part of one contiguous 1 KB store
// of the wave (and each 4-byte load part of a contiguous 256-byte load).
constexpr int kDequantChunk = 2048;

__global__ void __launch_bounds__(kDequantThreads)
nf4_dequant_kernel(const uint8_t *__restrict__ packed, const float *__restrict__ absmax,
                   const float *__restrict__ code, uint16_t *__restrict__ out, int64_t numel,
                   int32_t blocksize) {
  __shared__ float s_code[16];
  if (threadIdx.x < 16) s_code[threadIdx.x] = code[threadIdx.x];
  __syncthreads();

  const int lane = threadIdx.x & (kWave - 1);
  const int64_t nchunk = numel / kDequantChunk;
  const int64_t waves = (int64_t)gridDim.x * (kDequantThreads / kWave);
  for (int64_t c = (int64_t)blockIdx.x * (kDequantThreads / kWave) + (threadIdx.x >> 6); c < nchunk;
       c += waves) {
    const int64_t base = c * kDequantChunk;
    uint32_t q[4];
    float a[4];
#pragma unroll
    for (int s = 0; s < 4; ++s) {
      const int64_t v0 = base + 512 * s + 8 * lane;
      q[s] = *reinterpret_cast<const uint32_t *>(packed + v0 / 2);
      a[s] = absmax[v0 / blocksize];  // blocksize is a multiple of 32: one block per 8 values
    }
#pragma unroll
    for (int s = 0; s < 4; ++s) {
      uint32_t o[4];
#pragma unroll
      for (int b = 0; b < 4; ++b) {
        const uint32_t byte = (q[s] >> (8 * b)) & 0xffu;
        o[b] = pack_bf16x2(s_code[byte >> 4] * a[s], s_code[byte & 15u] * a[s]);
      }
      *reinterpret_cast<uint4 *>(out + base + 512 * s + 8 * lane) = make_uint4(o[0], o[1], o[2], o[3]);
    }
  }
  // Tail: fewer than one chunk left (numel is even), two values per thread of workgroup 0.
  if (blockIdx.x == 0) {
    for (int64_t i = nchunk * kDequantChunk + 2 * threadIdx.x; i < numel; i += 2 * kDequantThreads) {
      const uint32_t byte = packed[i / 2];
      out[i] = f32_to_bf16(s_code[byte >> 4] * absmax[i / blocksize]);
      out[i + 1] = f32_to_bf16(s_code[byte & 15u] * absmax[(i + 1) / blocksize]);
    }
  }
}

constexpr int kQuantThreads = 256;

// Blocksize-64 quantisation, eight lanes per block: lane l of a wave loads the 8 bf16 values
// at 8*l of the wave's 512-value chunk (one contiguous 1 KB load per wave), the block's
// absmax is the max over its 8 lanes (xor shuffles), and each lane packs its 8 values into
// 4 bytes (one contiguous 256-byte store per wave).  Same arithmetic as the per-block kernel
// below: q = number of codebook midpoints strictly below w * (1 / absmax), in fp32.
constexpr int kQuant64Chunk = 512;

__global__ void __launch_bounds__(kQuantThreads)
nf4_quantize64_kernel(const uint16_t *__restrict__ w, int64_t nchunk,
                      const float *__restrict__ code, uint8_t *__restrict__ packed,
                      float *__restrict__ absmax) {
  __shared__ float s_mid[16];
  if (threadIdx.x < 15) s_mid[threadIdx.x] = (code[threadIdx.x] + code[threadIdx.x + 1]) * 0.5f;
  __syncthreads();
  float mid[15];
#pragma unroll
  for (int m = 0; m < 15; ++m) mid[m] = s_mid[m];
  const int lane = threadIdx.x & (kWave - 1);
  const int64_t waves = (int64_t)gridDim.x * (kQuantThreads / kWave);
  for (int64_t c = (int64_t)blockIdx.x * (kQuantThreads / kWave) + (threadIdx.x >> 6); c < nchunk;
       c += waves) {
    const int64_t v0 = c * kQuant64Chunk + 8 * lane;
    const u32x4 raw = *reinterpret_cast<const u32x4 *>(w + v0);
    float x[8];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const uint32_t word = raw[i];
      x[2 * i] = bf16lo_to_f32(word);
      x[2 * i + 1] = bf16hi_to_f32(word);
    }
    float amax = 0.0f;
#pragma unroll
    for (int i = 0; i < 8; ++i) amax = fmaxf(amax, fabsf(x[i]));
#pragma unroll
    for (int off = 1; off < 8; off <<= 1) amax = fmaxf(amax, __shfl_xor(amax, off, kWave));
    if ((lane & 7) == 0) absmax[v0 / 64] = amax;
    const float r = amax > 0.0f ? 1.0f / amax : 0.0f;
    uint32_t out = 0;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const float y = x[i] * r;
      uint32_t q = 0;
#pragma unroll
      for (int m = 0; m < 15; ++m) q += y > mid[m] ? 1u : 0u;
      // value 2j in the high nibble of byte j
      out |= q << (8 * (i >> 1) + ((i & 1) ? 0 : 4));
    }
    *reinterpret_cast<uint32_t *>(packed + v0 / 2) = out;
  }
}

// One thread per quantisation block: any blocksize, partial last block.
__global__ void __launch_bounds__(kQuantThreads)
nf4_quantize_kernel(const uint16_t *__restrict__ w, int64_t numel, int32_t blocksize,
                    const float *__restrict__ code, uint8_t *__restrict__ packed,
                    float *__restrict__ absmax) {
  __shared__ float s_mid[15];
  if (threadIdx.x < 15) s_mid[threadIdx.x] = (code[threadIdx.x] + code[threadIdx.x + 1]) * 0.5f;
  __syncthreads();
  const int64_t nblocks = (numel + blocksize - 1) / blocksize;
  const int64_t b = (int64_t)blockIdx.x * kQuantThreads + threadIdx.x;
  if (b >= nblocks) return;
  const int64_t lo = b * blocksize;
  const int64_t hi = lo + blocksize < numel ? lo + blocksize : numel;
  float amax = 0.0f;
  for (int64_t i = lo; i < hi; ++i) amax = fmaxf(amax, fabsf(bf16_to_f32(w[i])));
  absmax[b] = amax;
  const float r = amax > 0.0f ? 1.0f / amax : 0.0f;
  for (int64_t i = lo; i < hi; i += 2) {
    int q[2];
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const float x = bf16_to_f32(w[i + j]) * r;
      int c = 0;
#pragma unroll
      for (int m = 0; m < 15; ++m) c += x > s_mid[m];
      q[j] = c;
    }
    packed[i / 2] = (uint8_t)((q[0] << 4) | q[1]);
  }
}

constexpr int kExpandThreads = 256;

// Nested (double-quantised) absmax: the fp32 block scales stored as 8-bit indices into a
// 256-entry code, with one fp32 scale per group of blocksize2 indices and a common offset.
// out[i] = code2[q[i]] * absmax2[i / blocksize2] + offset (a product, then a sum, each
// rounded in fp32 -- bitsandbytes' dequantize_blockwise of the absmax, then += offset).
__global__ void __launch_bounds__(kExpandThreads)
expand_absmax_kernel(const uint8_t *__restrict__ q, const float *__restrict__ absmax2,
                     const float *__restrict__ code2, float offset, int64_t n, int32_t blocksize2,
                     float *__restrict__ out) {
  __shared__ float s_code[256];
  s_code[threadIdx.x] = code2[threadIdx.x];
  __syncthreads();
  const int64_t i = (int64_t)blockIdx.x * kExpandThreads + threadIdx.x;
  if (i >= n) return;
  const float v = s_code[q[i]] * absmax2[i / blocksize2];
  out[i] = v + offset;
}

}  // namespace
}  // namespace moe

extern "C" int moe_nf4_expand_absmax(const void *absmax_u8, const void *absmax2_f32,
                                     const void *code2_f32, float offset, int64_t n,
                                     int32_t blocksize2, void *out_f32, void *stream) {
  MOE_REQUIRE(n >= 0, "n must be non-negative (got %lld)", (long long)n);
  MOE_REQUIRE(blocksize2 > 0, "blocksize2 must be positive (got %d)", blocksize2);
  if (n == 0) return MOE_STATUS_OK;
  MOE_REQUIRE(absmax_u8 && absmax2_f32 && code2_f32 && out_f32, "null device pointer");
  const int64_t grid = (n + moe::kExpandThreads - 1) / moe::kExpandThreads;
  MOE_REQUIRE(grid <= 0x7fffffff, "n too large");
  hipLaunchKernelGGL(moe::expand_absmax_kernel, dim3((unsigned)grid), dim3(moe::kExpandThreads), 0,
                     (hipStream_t)stream, (const uint8_t *)absmax_u8, (const float *)absmax2_f32,
                     (const float *)code2_f32, offset, n, blocksize2, (float *)out_f32);
  MOE_LAUNCH_CHECK();
  return MOE_STATUS_OK;
}

extern "C" int moe_nf4_dequant_bf16(const void *packed, const void *absmax, const void *code16,
                                    void *out_bf16, int64_t numel, int32_t blocksize,
                                    void *stream) {
  MOE_REQUIRE(numel >= 0 && numel % 2 == 0, "numel must be even and non-negative (got %lld)",
              (long long)numel);
  MOE_REQUIRE(blocksize > 0 && blocksize % 32 == 0,
              "blocksize must be a positive multiple of 32 (got %d)", blocksize);
  if (numel == 0) return MOE_STATUS_OK;
  MOE_REQUIRE(packed && absmax && code16 && out_bf16, "null device pointer");
  MOE_REQUIRE(((uintptr_t)packed % 16) == 0 && ((uintptr_t)out_bf16 % 16) == 0,
              "packed and out must be 16-byte aligned");
  const int64_t nchunk = numel / moe::kDequantChunk;
  int64_t blocks = (nchunk + (moe::kDequantThreads / moe::kWave) - 1) / (moe::kDequantThreads / moe::kWave);
  const int64_t cap = (int64_t)moe::device_cu_count() * 8;
  if (blocks > cap) blocks = cap;
  if (blocks < 1) blocks = 1;
  hipLaunchKernelGGL(moe::nf4_dequant_kernel, dim3((unsigned)blocks), dim3(moe::kDequantThreads),
                     0, (hipStream_t)stream, (const uint8_t *)packed, (const float *)absmax,
                     (const float *)code16, (uint16_t *)out_bf16, numel, blocksize);
  MOE_LAUNCH_CHECK();
  return MOE_STATUS_OK;
}

extern "C" int moe_nf4_quantize_bf16(const void *w_bf16, int64_t numel, int32_t blocksize,
                                     const void *code16, void *packed_out, void *absmax_out,
                                     void *stream) {
  MOE_REQUIRE(numel >= 0 && numel % 2 == 0, "numel must be even and non-negative (got %lld)",
              (long long)numel);
  MOE_REQUIRE(blocksize >= 2 && blocksize <= 4096 && blocksize % 2 == 0,
              "blocksize must be even and in [2, 4096] (got %d)", blocksize);
  if (numel == 0) return MOE_STATUS_OK;
  MOE_REQUIRE(w_bf16 && code16 && packed_out && absmax_out, "null device pointer");
  if (blocksize == 64 && numel % moe::kQuant64Chunk == 0 && ((uintptr_t)w_bf16 % 16) == 0 &&
      ((uintptr_t)packed_out % 4) == 0 && ((uintptr_t)absmax_out % 4) == 0) {
    const int64_t nchunk = numel / moe::kQuant64Chunk;
    int64_t blocks = (nchunk + (moe::kQuantThreads / moe::kWave) - 1) / (moe::kQuantThreads / moe::kWave);
    const int64_t cap = (int64_t)moe::device_cu_count() * 8;
    blocks = blocks > cap ? cap : blocks;
    hipLaunchKernelGGL(moe::nf4_quantize64_kernel, dim3((unsigned)blocks), dim3(moe::kQuantThreads),
                       0, (hipStream_t)stream, (const uint16_t *)w_bf16, nchunk,
                       (const float *)code16, (uint8_t *)packed_out, (float *)absmax_out);
    MOE_LAUNCH_CHECK();
    return MOE_STATUS_OK;
  }
  const int64_t nblocks = (numel + blocksize - 1) / blocksize;
  const int64_t grid = (nblocks + moe::kQuantThreads - 1) / moe::kQuantThreads;
  MOE_REQUIRE(grid <= 0x7fffffff, "numel too large");
  hipLaunchKernelGGL(moe::nf4_quantize_kernel, dim3((unsigned)grid), dim3(moe::kQuantThreads), 0,
                     (hipStream_t)stream, (const uint16_t *)w_bf16, numel, blocksize,
                     (const float *)code16, (uint8_t *)packed_out, (float *)absmax_out);
  MOE_LAUNCH_CHECK();
  return MOE_STATUS_OK;
}
