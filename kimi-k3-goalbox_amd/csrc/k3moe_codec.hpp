// MXFP4 encoder: pack_mxfp4 of megabench/tasks/quantization.py:13-37 on the
// GPU, bit for bit with its torch CPU chain (fp32 throughout).
//
// Per block of 32 values along the last axis:
//   e      = ceil(log2(max(max|x| / 6, 2^-126))), clamped to [-126, 127]
//            (:24-26). log2 is torch's fp32 logarithm, which rounds to the
//            nearest fp32: for a quotient v = 2^n (1 + j 2^-23) with j > 0 the
//            exact ceiling is n + 1, but when log2(v) - n is below half an
//            fp32 step of n the rounded logarithm is n itself and the ceiling
//            stays n. That happens only for small j (j < 23 at |n| < 128), so
//            those quotients take a float64 log2 rounded once to fp32, and
//            every other quotient the exact ceiling from its bits.
//   a      = x * 2^-e as an IEEE fp32 product (:27; subnormal products are
//            rounded, as torch's ldexp rounds them);
//   code   = number of boundaries (0.25 0.75 1.25 1.75 2.5 3.5 5.0) below |a|,
//            plus one at the ties 0.75, 1.75 and 3.5 whose lower code is odd
//            (round to nearest, ties to the even code, :28-34); NaN takes 7
//            (bucketize puts NaN last); | 8 when a < 0 (:35);
//   bytes  = code[2j] | code[2j+1] << 4, scale byte e + 127 (:36-37).
// A block holding a NaN follows torch on x86: its NaN maximum converts to
// int32 as INT_MIN, so the scale byte wraps to 127 and ldexp scales by
// 2^INT_MIN = 0 (NaN and infinite elements then take code 7, finite ones 0).
//
// Layout: 4 lanes per block, lane s of the group holding elements 8s .. 8s+7
// (one 16-byte load of bf16 / fp16, two of fp32), so a wave reads 16
// consecutive blocks with contiguous 16-byte loads and writes their 256 packed
// bytes with contiguous 4-byte stores and their 16 scale bytes with one byte
// store per block; the block maximum is two xor-shuffles.
// HBM-bound: per block 32 input values in, 17 bytes out.
#pragma once

#include "k3moe_device.hpp"

namespace k3moe {

constexpr int kEncThreads = 256;

// The block exponent e (before the +127 bias) of a finite or infinite block
// maximum, as torch's chain computes it (see the file comment).
__device__ __forceinline__ int mx_block_exponent(float amax) {
  float v = amax / 6.0f;  // IEEE fp32 division
  if (!(v >= 0x1p-126f)) v = 0x1p-126f;
  const uint32_t b = __float_as_uint(v);
  const int n = (int)(b >> 23) - 127;
  if (n > 127) return 127;  // infinite maximum
  const uint32_t j = b & 0x7FFFFFu;
  int e = j == 0u ? n : n + 1;
  if (j != 0u && j < 64u && n != 0) e = (int)ceilf((float)log2((double)v));
  return e < -126 ? -126 : (e > 127 ? 127 : e);
}

// E2M1 code of one block-normalised value (ties to the even code, NaN -> 7).
__device__ __forceinline__ uint32_t e2m1_code(float a) {
  const float m = fabsf(a);
  uint32_t c = (uint32_t)(m > 0.25f) + (uint32_t)(m > 0.75f) + (uint32_t)(m > 1.25f) + (uint32_t)(m > 1.75f) +
               (uint32_t)(m > 2.5f) + (uint32_t)(m > 3.5f) + (uint32_t)(m > 5.0f);
  c += (uint32_t)((m == 0.75f) | (m == 1.75f) | (m == 3.5f));
  if (m != m) c = 7u;
  return c | (a < 0.f ? 8u : 0u);
}

// 2^-e as an fp32 value, exact for e in [-126, 127] (2^-127 is subnormal).
__device__ __forceinline__ float pow2_neg(int e) {
  return e == 127 ? __uint_as_float(0x00400000u) : __uint_as_float((uint32_t)(127 - e) << 23);
}

// in_dtype: K3MOE_DTYPE_F32 / _BF16 / _F16 (values converted to fp32 exactly)
__global__ __launch_bounds__(kEncThreads) void k_encode(const void *__restrict__ in, int in_dtype, int64_t n_blocks,
                                                        uint8_t *__restrict__ blocks, uint8_t *__restrict__ scales) {
  const int s = threadIdx.x & 3;
  const int64_t stride = (int64_t)gridDim.x * (kEncThreads / 4);
  for (int64_t blk = (int64_t)blockIdx.x * (kEncThreads / 4) + (threadIdx.x >> 2); blk < n_blocks; blk += stride) {
    float v[8];
    if (in_dtype == 1) {  // fp32
      const float *src = reinterpret_cast<const float *>(in) + blk * 32 + 8 * s;
      const u32x4 w0 = *reinterpret_cast<const u32x4 *>(src), w1 = *reinterpret_cast<const u32x4 *>(src + 4);
#pragma unroll
      for (int t = 0; t < 4; ++t) {
        v[t] = __uint_as_float(w0[t]);
        v[4 + t] = __uint_as_float(w1[t]);
      }
    } else {
      const u32x4 w = *reinterpret_cast<const u32x4 *>(reinterpret_cast<const uint16_t *>(in) + blk * 32 + 8 * s);
#pragma unroll
      for (int t = 0; t < 8; ++t) {
        const uint32_t h = (w[t >> 1] >> (16 * (t & 1))) & 0xFFFFu;
        v[t] = in_dtype == 0 ? __uint_as_float(h << 16) : (float)__builtin_bit_cast(_Float16, (uint16_t)h);
      }
    }
    float amax = 0.f;
    int nan = 0;
#pragma unroll
    for (int t = 0; t < 8; ++t) {
      amax = fmaxf(amax, fabsf(v[t]));
      nan |= v[t] != v[t];
    }
#pragma unroll
    for (int m = 1; m < 4; m <<= 1) {
      amax = fmaxf(amax, shfl_xor(amax, m));
      nan |= shfl_xor(nan, m);
    }
    uint32_t sbyte;
    float step;
    if (nan) {
      sbyte = 127u;
      step = 0.f;
    } else {
      const int e = mx_block_exponent(amax);
      sbyte = (uint32_t)(e + 127);
      step = pow2_neg(e);
    }
    uint32_t packed = 0u;
#pragma unroll
    for (int t = 0; t < 8; ++t) packed |= e2m1_code(__fmul_rn(v[t], step)) << (4 * t);
    *reinterpret_cast<uint32_t *>(blocks + blk * 16 + 4 * s) = packed;
    if (s == 0) scales[blk] = (uint8_t)sbyte;
  }
}

}  // namespace k3moe
