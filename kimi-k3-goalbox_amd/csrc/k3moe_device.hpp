// Device-side building blocks shared by the k3moe kernels (gfx950 only).
//
// MFMA tile convention (v_mfma_f32_16x16x32_bf16, one wave of 64 lanes):
//   A (16 weight rows x 32 k):  lane l holds row (l % 16), k = 8*(l / 16) + e, e = 0..7
//   B (32 k x 16 token cols):   lane l holds col (l % 16), k = 8*(l / 16) + e
//   D (16 x 16 fp32):           lane l holds col (l % 16), rows 4*(l / 16) + v, v = 0..3
// A and B use the same (lane group, element) -> k assignment, so any
// consistent k permutation gives the same dot products.
//
// One "k-step" covers 128 consecutive k (four 32-wide MXFP4 blocks): lane
// group q = l / 16 owns block 4*step + q of its row and feeds its 32 values
// to four MFMAs (kk = 0..3, elements 8*kk .. 8*kk+7 of the block).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace k3moe {

typedef __attribute__((ext_vector_type(8))) __bf16 bf16x8;
typedef __attribute__((ext_vector_type(2))) __bf16 bf16x2;
typedef __attribute__((ext_vector_type(4))) float f32x4;
typedef __attribute__((ext_vector_type(4))) uint32_t u32x4;
typedef __attribute__((ext_vector_type(2))) uint32_t u32x2;

constexpr int kWave = 64;
constexpr int kBlockK = 32;  // MXFP4 block (quantization.py:10)
constexpr int kStepK = 128;  // k covered by one k-step of a wave

__device__ __forceinline__ int lane_id() { return __lane_id(); }
// The wave's index in the workgroup, as a value the compiler knows to be
// wave-uniform: loops and branches on it then use scalar control flow rather
// than exec-mask loops (whose merged paths also make the wait counts of the
// loads in them conservative).
__device__ __forceinline__ int wave_id() { return __builtin_amdgcn_readfirstlane((int)threadIdx.x >> 6); }

// ---------------------------------------------------------------- bf16 bits --

// FP32 -> BF16 with round-to-nearest-even (the hardware conversion); NaN -> a quiet NaN.
__device__ __forceinline__ uint16_t f32_to_bf16_bits(float f) {
  return __builtin_bit_cast(uint16_t, (__bf16)f);  // v_cvt_pk_bf16_f32: round to nearest even
}

__device__ __forceinline__ float bf16_bits_to_f32(uint32_t b) { return __uint_as_float(b << 16); }

// Round an FP32 value to the nearest BF16 and return it as FP32.
__device__ __forceinline__ float round_bf16(float f) { return bf16_bits_to_f32(f32_to_bf16_bits(f)); }

// ------------------------------------------------------------ MXFP4 decode --

// Exact FP32 bits of one E2M1 code scaled by 2^(s-127) (OCP MX v1.0):
// sign bit 3, exponent bits 2..1 (bias 1), mantissa bit 0; E8M0 255 is NaN.
__device__ __forceinline__ uint32_t mxfp4_bits(uint32_t code, uint32_t s) {
  if (s == 255u) return 0x7FC00000u;
  uint32_t sign = (code & 8u) << 28;
  uint32_t e = (code >> 1) & 3u, m = code & 1u;
  if (e == 0u && m == 0u) return sign;
  // unscaled value as (biased exponent, 1-bit mantissa): 0.5 = 2^-1, else 2^(e-1)(1+m/2)
  int32_t be = (e == 0u) ? 126 : (int32_t)(e + 126u);
  uint32_t mant = (e == 0u) ? 0u : (m << 22);
  int32_t ne = be + (int32_t)s - 127;
  if (ne >= 255) return sign | 0x7F800000u;
  if (ne >= 1) return sign | ((uint32_t)ne << 23) | mant;
  uint32_t sig = (1u << 23) | mant;  // subnormal result: exact right shift
  return sign | (sig >> (1 - ne));
}

// E8M0 byte placed in the exponent field of an FP32 scale operand.
__device__ __forceinline__ float e8m0_to_f32(uint32_t s) { return __uint_as_float(s << 23); }

// v_cvt_scalef32_pk_{bf16,f32}_fp4 reads only the exponent field of its FP32
// scale operand and reproduces the exact decode (subnormal and overflowing
// products included) for every E8M0 byte except 255, where it returns a
// negative NaN instead of the canonical quiet NaN; measured over all 256 x 256
// (byte, scale) pairs on MI355X. Byte 255 therefore takes the bit construction.
__device__ __forceinline__ bool scale_is_plain(uint32_t s) { return s != 255u; }

// Eight E2M1 codes (one 32-bit word, element order = nibble order, low nibble
// first) scaled by `scale` -> bf16x8 via v_cvt_scalef32_pk_bf16_fp4.
__device__ __forceinline__ bf16x8 fp4x8_to_bf16(uint32_t w, float scale) {
  bf16x2 p0 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(w, scale, 0);
  bf16x2 p1 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(w, scale, 1);
  bf16x2 p2 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(w, scale, 2);
  bf16x2 p3 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(w, scale, 3);
  bf16x8 r;
  r[0] = p0[0]; r[1] = p0[1]; r[2] = p1[0]; r[3] = p1[1];
  r[4] = p2[0]; r[5] = p2[1]; r[6] = p3[0]; r[7] = p3[1];
  return r;
}

// Exact decode of eight codes to bf16 by bit construction (any scale byte).
__device__ __forceinline__ bf16x8 fp4x8_to_bf16_exact(uint32_t w, uint32_t s) {
  uint32_t packed[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    uint32_t lo = mxfp4_bits((w >> (8 * i)) & 15u, s) >> 16;
    uint32_t hi = mxfp4_bits((w >> (8 * i + 4)) & 15u, s) >> 16;
    packed[i] = lo | (hi << 16);
  }
  u32x4 v = {packed[0], packed[1], packed[2], packed[3]};
  return __builtin_bit_cast(bf16x8, v);
}

// The 32 values of one MXFP4 block (16 bytes) as four bf16x8 MFMA operands:
// hardware conversion for scale bytes 0..254, bit construction for 255.
__device__ __forceinline__ void convert_block(const u32x4 &w, uint32_t s, bf16x8 out[4]) {
  if (scale_is_plain(s)) {
    float sc = e8m0_to_f32(s);
    out[0] = fp4x8_to_bf16(w[0], sc);
    out[1] = fp4x8_to_bf16(w[1], sc);
    out[2] = fp4x8_to_bf16(w[2], sc);
    out[3] = fp4x8_to_bf16(w[3], sc);
  } else {
    out[0] = fp4x8_to_bf16_exact(w[0], s);
    out[1] = fp4x8_to_bf16_exact(w[1], s);
    out[2] = fp4x8_to_bf16_exact(w[2], s);
    out[3] = fp4x8_to_bf16_exact(w[3], s);
  }
}

// Same conversion with the hardware path for every scale byte, for the GEMMs:
// scale 255 then yields NaN of the other sign, which propagates to the same
// NaN outputs.
__device__ __forceinline__ void convert_block_fast(const u32x4 &w, uint32_t s, bf16x8 out[4]) {
  const float sc = e8m0_to_f32(s);
  out[0] = fp4x8_to_bf16(w[0], sc);
  out[1] = fp4x8_to_bf16(w[1], sc);
  out[2] = fp4x8_to_bf16(w[2], sc);
  out[3] = fp4x8_to_bf16(w[3], sc);
}

__device__ __forceinline__ bf16x8 as_bf16x8(const u32x4 &v) { return __builtin_bit_cast(bf16x8, v); }

__device__ __forceinline__ f32x4 mfma16(const bf16x8 &a, const bf16x8 &b, const f32x4 &c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}

__device__ __forceinline__ u32x4 load16(const void *p) { return *reinterpret_cast<const u32x4 *>(p); }

// Raw buffer resource over [base, base + bytes) (gfx9 descriptor word 3): a
// load at an offset past the end returns zero and touches no memory, which is
// how inactive lanes skip their operand loads without branching.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void *base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(base), 0, (int)bytes, 0x00020000);
}

constexpr uint32_t kOffNone = 0x80000000u;  // a buffer offset past every resource used here

__device__ __forceinline__ u32x4 bload16(__amdgpu_buffer_rsrc_t r, uint32_t off) {
  return __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(r, (int)off, 0, 0));
}

// Streaming weight load. A wave's 16-byte loads cover half of each 128-byte
// line (4 blocks of 16 rows); the other half is loaded one k-step later, so
// the line must stay in L2 in between: plain loads, not non-temporal ones.
__device__ __forceinline__ u32x4 load16_nt(const void *p) { return *reinterpret_cast<const u32x4 *>(p); }

// Device-coherent stores (cache policy sc1, the encoding of an agent-scope
// atomic store): written through past the XCD's L2, so data that other
// workgroups read after a grid barrier needs no L2 write-back at the barrier,
// only the completion of the stores (vmcnt). `r` is a buffer resource over
// the destination array, `off` a byte offset.
constexpr int kCpolDevice = 16;

__device__ __forceinline__ void st_dev32(__amdgpu_buffer_rsrc_t r, uint32_t off, uint32_t v) {
  __builtin_amdgcn_raw_buffer_store_b32(v, r, off, 0, kCpolDevice);
}
__device__ __forceinline__ void st_dev64(__amdgpu_buffer_rsrc_t r, uint32_t off, u32x2 v) {
  __builtin_amdgcn_raw_buffer_store_b64(v, r, off, 0, kCpolDevice);
}
__device__ __forceinline__ void st_dev128(__amdgpu_buffer_rsrc_t r, uint32_t off, u32x4 v) {
  __builtin_amdgcn_raw_buffer_store_b128(v, r, off, 0, kCpolDevice);
}

// Reads the first Bytes of the kernel-argument segment with ten independent
// scalar loads (every 64-byte line, whatever the segment's alignment, and its
// last dword) and one wait, and returns the segment's address. A kernel whose
// arguments do not fit its scalar registers reads them in a chain of load /
// wait steps; reading them through the returned address (opaque to the
// compiler, so no argument load is scheduled before the touch) makes every
// step of that chain hit the scalar cache instead of missing to memory.
template <int Bytes>
__device__ __forceinline__ uint64_t touch_kernargs() {
  static_assert(Bytes >= 8 && Bytes <= 580 && Bytes % 4 == 0, "ten loads cover at most 580 bytes");
  constexpr int last = Bytes - 4;
  uint64_t base = reinterpret_cast<uint64_t>(__builtin_amdgcn_kernarg_segment_ptr());
  uint32_t t0, t1, t2, t3, t4, t5, t6, t7, t8, t9;
  asm volatile(
      "s_load_dword %0, %10, %11\n\t"
      "s_load_dword %1, %10, %12\n\t"
      "s_load_dword %2, %10, %13\n\t"
      "s_load_dword %3, %10, %14\n\t"
      "s_load_dword %4, %10, %15\n\t"
      "s_load_dword %5, %10, %16\n\t"
      "s_load_dword %6, %10, %17\n\t"
      "s_load_dword %7, %10, %18\n\t"
      "s_load_dword %8, %10, %19\n\t"
      "s_load_dword %9, %10, %20\n\t"
      "s_waitcnt lgkmcnt(0)"
      : "=&s"(t0), "=&s"(t1), "=&s"(t2), "=&s"(t3), "=&s"(t4), "=&s"(t5), "=&s"(t6), "=&s"(t7), "=&s"(t8),
        "=&s"(t9), "+s"(base)
      : "n"(0), "n"(64 < last ? 64 : last), "n"(128 < last ? 128 : last), "n"(192 < last ? 192 : last),
        "n"(256 < last ? 256 : last), "n"(320 < last ? 320 : last), "n"(384 < last ? 384 : last),
        "n"(448 < last ? 448 : last), "n"(512 < last ? 512 : last), "n"(last));
  return base;
}

// A copy of the T at constant-memory address `addr` (the kernel-argument
// segment), read as 32-bit words: the compiler keeps the fields it uses in
// scalar registers or reloads them with scalar loads.
template <class T>
__device__ __forceinline__ T load_const(uint64_t addr) {
  static_assert(sizeof(T) % 4 == 0, "whole words");
  typedef const uint32_t __attribute__((address_space(4))) cu32;
  const cu32 *src = reinterpret_cast<const cu32 *>(addr);
  T v;
  uint32_t *dst = reinterpret_cast<uint32_t *>(&v);
#pragma unroll
  for (int j = 0; j < (int)(sizeof(T) / 4); ++j) dst[j] = src[j];
  return v;
}

// The pointer stored at constant-memory address `addr` (the kernel-argument
// segment), read as a global-memory pointer: the compiler's address-space
// inference then emits global loads and stores through it and everything
// derived from it, not flat ones (a flat access also counts as an LDS access,
// so waits for LDS results would wait for it too).
template <class T>
__device__ __forceinline__ T *global_field(uint64_t addr) {
  typedef T __attribute__((address_space(1))) GT;
  GT *const __attribute__((address_space(4))) *slot =
      reinterpret_cast<GT *const __attribute__((address_space(4))) *>(addr);
  return (T *)*slot;
}

// Address of the next instruction.
__device__ __forceinline__ uint64_t program_counter() {
  uint64_t pc;
  asm volatile("s_getpc_b64 %0" : "=s"(pc));
  return pc;
}

// Device-coherent 8-byte load (sc1).
__device__ __forceinline__ u32x2 bload8_dev(__amdgpu_buffer_rsrc_t r, uint32_t off) {
  return __builtin_bit_cast(u32x2, __builtin_amdgcn_raw_buffer_load_b64(r, (int)off, 0, kCpolDevice));
}

// Device-coherent 16-byte load (sc1): sees device-coherent stores of other
// workgroups without an L2 invalidate.
__device__ __forceinline__ u32x4 bload16_dev(__amdgpu_buffer_rsrc_t r, uint32_t off) {
  return __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(r, (int)off, 0, kCpolDevice));
}

// Wait until every vector memory operation of this wave has completed.
__device__ __forceinline__ void wait_vmem() { __builtin_amdgcn_s_waitcnt(0x0F70); }

// Waits until at most N of this wave's vector memory operations are in flight
// (direct-to-LDS loads are not tracked by the compiler's own waits).
template <int N>
__device__ __forceinline__ void wait_vm() {
  asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}

// Workgroup barrier for hand-offs through LDS, without the memory fence of
// __syncthreads (whose release would also wait for the global loads still in
// flight for later steps). It orders LDS only: each wave's LDS reads and
// writes before it are complete (lgkmcnt) at it. Data loaded directly to LDS
// must be waited for (wait_vm) before it.
__device__ __forceinline__ void ring_barrier() {
  asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
}

// 16 (or 4) bytes per lane from global memory to LDS: lane L's bytes land at
// dst + L * size; dst is the same for the whole wave. Aux is the cache policy
// (kCpolDevice: a device-coherent read). The compiler counts these loads in
// vmcnt but does not wait for them before LDS reads: wait_vm first.
template <int Size, int Aux = 0>
__device__ __forceinline__ void load_lds(const void *src, char *dst) {
  static_assert(Size == 16 || Size == 4, "16- or 4-byte lanes");
  typedef __attribute__((address_space(3))) void lds_void;
  if constexpr (Size == 16)
    __builtin_amdgcn_global_load_lds(src, (lds_void *)dst, 16, 0, Aux);
  else
    __builtin_amdgcn_global_load_lds(src, (lds_void *)dst, 4, 0, Aux);
}

// ------------------------------------------------------------- activations --

// SiTU (kimi.py:194-196) on bf16-rounded gate/up values, in FP32 with the
// reference's operation order: ((4 tanh(g/4)) sigmoid(g)) (25 tanh(u/25)).
__device__ __forceinline__ float act_situ(float g, float u) {
  float sig = 1.0f / (1.0f + expf(-g));
  float a = __fmul_rn(4.0f, tanhf(g / 4.0f));
  a = __fmul_rn(a, sig);
  float b = __fmul_rn(25.0f, tanhf(u / 25.0f));
  return __fmul_rn(a, b);
}

// silu(g) u (distributed.py:184) in FP32.
__device__ __forceinline__ float act_silu(float g, float u) {
  float sig = 1.0f / (1.0f + expf(-g));
  return __fmul_rn(__fmul_rn(g, sig), u);
}

__device__ __forceinline__ float apply_act(int act, float g, float u) {
  return act == 0 ? act_situ(g, u) : act_silu(g, u);
}

// The same activations from the hardware's base-2 exponential and reciprocal
// (v_exp_f32, v_rcp_f32, about 1 ulp each) instead of the library's expf and
// tanhf, for the prefill GEMM's epilogue, where they are most of its time:
//   sigmoid(g) = 1 / (1 + e), or e / (1 + e) for g < 0, with e = 2^(-|g| log2 e),
//   tanh(y) = sign(y) (1 - e) / (1 + e) with e = 2^(-2 |y| log2 e), and for
//   |y| < 1/16, where 1 - e cancels, the Taylor series y - y^3/3 + 2 y^5/15
//   (the next term is below 2^-27 of y there).
// Relative error a few fp32 ulps (GPU test against a float64 reference), far
// below the bf16 rounding of h that follows.
constexpr float kLog2e = 1.44269504088896340736f;  // log2(e)
__device__ __forceinline__ float fast_sigmoid(float g) {
  // e = exp(-|g|) in (0, 1]: sigmoid(g) = 1 / (1 + e) for g >= 0, e / (1 + e) below (no overflow)
  const float e = __builtin_amdgcn_exp2f(__fmul_rn(-fabsf(g), kLog2e));
  const float r = __builtin_amdgcn_rcpf(__fadd_rn(1.0f, e));
  return g >= 0.0f ? r : __fmul_rn(e, r);
}
__device__ __forceinline__ float fast_tanh(float y) {
  const float a = fabsf(y), y2 = __fmul_rn(y, y);
  const float poly = __fmul_rn(y, __fsub_rn(1.0f, __fmul_rn(y2, __fsub_rn(1.0f / 3.0f, __fmul_rn(y2, 2.0f / 15.0f)))));
  const float e = __builtin_amdgcn_exp2f(__fmul_rn(-2.0f * kLog2e, a));
  const float t = __fmul_rn(__fsub_rn(1.0f, e), __builtin_amdgcn_rcpf(__fadd_rn(1.0f, e)));
  return a < 0.0625f ? poly : copysignf(t, y);
}
__device__ __forceinline__ float fast_act(int act, float g, float u) {
  const float sig = fast_sigmoid(g);
  if (act == 0) {
    const float a = __fmul_rn(__fmul_rn(4.0f, fast_tanh(__fmul_rn(g, 0.25f))), sig);
    return __fmul_rn(a, __fmul_rn(25.0f, fast_tanh(__fmul_rn(u, 0.04f))));
  }
  return __fmul_rn(__fmul_rn(g, sig), u);
}

// apply_act for row l & 7 of a wave, lanes 0-7 returning it, with its
// transcendental factors spread over lanes: lane l computes factor l >> 3 of
// row l & 7 (0: sigmoid(g), 1: tanh(g/4), 2: tanh(u/25)) and lanes 0-7 combine
// them with the same operations in the same order as act_situ / act_silu, so
// the result is the same bit for bit. g, u: row (l & 7)'s bf16-rounded gate and
// up values in every lane. Every lane must call it.
__device__ __forceinline__ float act_parts(int act, float g, float u) {
  const int l = __lane_id(), f = l >> 3;
  float part = 0.f;
  if (f == 0) part = 1.0f / (1.0f + expf(-g));
  else if (f == 1) part = tanhf(g / 4.0f);
  else if (f == 2) part = tanhf(u / 25.0f);
  const float sig = __shfl(part, l & 7, kWave), tg = __shfl(part, 8 + (l & 7), kWave),
              tu = __shfl(part, 16 + (l & 7), kWave);
  if (act == 0) return __fmul_rn(__fmul_rn(__fmul_rn(4.0f, tg), sig), __fmul_rn(25.0f, tu));
  return __fmul_rn(__fmul_rn(g, sig), u);
}

// ----------------------------------------------------------- wave helpers --

template <typename T>
__device__ __forceinline__ T shfl_xor(T v, int mask) {
  return __shfl_xor(v, mask, kWave);
}

// DPP controls (GFX9): quad_perm [1,0,3,2] and [2,3,0,1], row_half_mirror,
// row_mirror, row_bcast:15, row_bcast:31.
constexpr int kDppQuadXor1 = 0xB1, kDppQuadXor2 = 0x4E, kDppHalfMirror = 0x141, kDppMirror = 0x140,
              kDppBcast15 = 0x142, kDppBcast31 = 0x143;

template <int Ctrl, int RowMask>
__device__ __forceinline__ uint32_t dpp(uint32_t v) {
  return (uint32_t)__builtin_amdgcn_update_dpp((int)v, (int)v, Ctrl, RowMask, 0xF, false);
}

// Wave-wide maximum / minimum of an unsigned value, returned to every lane:
// pairs inside quads, then half-rows and rows, then the row broadcasts fold
// rows 0..3 into lane 63.
__device__ __forceinline__ uint32_t wave_max_u32(uint32_t v) {
  v = max(v, dpp<kDppQuadXor1, 0xF>(v));
  v = max(v, dpp<kDppQuadXor2, 0xF>(v));
  v = max(v, dpp<kDppHalfMirror, 0xF>(v));
  v = max(v, dpp<kDppMirror, 0xF>(v));
  v = max(v, dpp<kDppBcast15, 0xA>(v));
  v = max(v, dpp<kDppBcast31, 0xC>(v));
  return (uint32_t)__builtin_amdgcn_readlane((int)v, 63);
}

// Wave-wide FP32 sum in a fixed order (pairs inside quads, half-rows, rows,
// then the row broadcasts into lane 63), returned to every lane.
__device__ __forceinline__ float wave_sum_f32(float v) {
  auto add = [](float a, uint32_t b) { return __fadd_rn(a, __uint_as_float(b)); };
  v = add(v, dpp<kDppQuadXor1, 0xF>(__float_as_uint(v)));
  v = add(v, dpp<kDppQuadXor2, 0xF>(__float_as_uint(v)));
  v = add(v, dpp<kDppHalfMirror, 0xF>(__float_as_uint(v)));
  v = add(v, dpp<kDppMirror, 0xF>(__float_as_uint(v)));
  const float b15 = __uint_as_float(dpp<kDppBcast15, 0xA>(__float_as_uint(v)));
  v = (__lane_id() & 16) ? __fadd_rn(v, b15) : v;
  const float b31 = __uint_as_float(dpp<kDppBcast31, 0xC>(__float_as_uint(v)));
  v = (__lane_id() & 32) ? __fadd_rn(v, b31) : v;
  return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 63));
}

__device__ __forceinline__ uint32_t wave_or_u32(uint32_t v) {
  v |= dpp<kDppQuadXor1, 0xF>(v);
  v |= dpp<kDppQuadXor2, 0xF>(v);
  v |= dpp<kDppHalfMirror, 0xF>(v);
  v |= dpp<kDppMirror, 0xF>(v);
  v |= dpp<kDppBcast15, 0xA>(v);
  v |= dpp<kDppBcast31, 0xC>(v);
  return (uint32_t)__builtin_amdgcn_readlane((int)v, 63);
}

__device__ __forceinline__ uint32_t wave_min_u32(uint32_t v) {
  v = min(v, dpp<kDppQuadXor1, 0xF>(v));
  v = min(v, dpp<kDppQuadXor2, 0xF>(v));
  v = min(v, dpp<kDppHalfMirror, 0xF>(v));
  v = min(v, dpp<kDppMirror, 0xF>(v));
  v = min(v, dpp<kDppBcast15, 0xA>(v));
  v = min(v, dpp<kDppBcast31, 0xC>(v));
  return (uint32_t)__builtin_amdgcn_readlane((int)v, 63);
}

// Order-preserving map of an FP32 value to uint32: larger float -> larger
// key; -0.0 and +0.0 share a key; every NaN maps above +inf (top-k treats NaN
// as the largest value).
__device__ __forceinline__ uint32_t ordered_key(float f) {
  uint32_t u = __float_as_uint(f);
  if ((u & 0x7FFFFFFFu) > 0x7F800000u) return 0xFFFFFFFFu;
  if (u == 0x80000000u) u = 0u;
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

// Value of lane `src` (wave-uniform) in every lane.
__device__ __forceinline__ uint32_t lane_u32(uint32_t v, int src) {
  return (uint32_t)__builtin_amdgcn_readlane((int)v, src);
}
__device__ __forceinline__ float lane_f32(float v, int src) {
  return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), src));
}

// Forced routes of token t (kimi.py:311-313), read by lanes l < k: *id gets
// the lane's expert id. Returns (wave-uniform) whether the row is valid: every
// id in [0, E) and the k ids distinct (kimi.py:364-367). An invalid row must
// not be used: its ids would index the expert tensors and the LDS lists.
__device__ __forceinline__ bool forced_route(const int64_t *routes, int t, int k, int E, int *id) {
  const int l = threadIdx.x & 63;
  const int64_t r = l < k ? routes[(size_t)t * k + l] : 0;
  bool bad = l < k && (r < 0 || r >= E);
  const int mine = (int)r;
  for (int j = 0; j < k; ++j) bad |= l < k && j < l && (int)lane_u32((uint32_t)mine, j) == mine;
  *id = mine;
  return __ballot(bad) == 0;
}

// One DPP step of a 64-bit wave maximum: max(v, v of the DPP source lane).
template <int Ctrl, int RowMask>
__device__ __forceinline__ uint64_t dpp_max_u64(uint64_t v) {
  const uint32_t lo = dpp<Ctrl, RowMask>((uint32_t)v), hi = dpp<Ctrl, RowMask>((uint32_t)(v >> 32));
  const uint64_t o = ((uint64_t)hi << 32) | lo;
  return o > v ? o : v;
}

// Wave-wide maximum of a 64-bit value, in every lane (same DPP pattern as wave_max_u32).
__device__ __forceinline__ uint64_t wave_max_u64(uint64_t v) {
  v = dpp_max_u64<kDppQuadXor1, 0xF>(v);
  v = dpp_max_u64<kDppQuadXor2, 0xF>(v);
  v = dpp_max_u64<kDppHalfMirror, 0xF>(v);
  v = dpp_max_u64<kDppMirror, 0xF>(v);
  v = dpp_max_u64<kDppBcast15, 0xA>(v);
  v = dpp_max_u64<kDppBcast31, 0xC>(v);
  return ((uint64_t)lane_u32((uint32_t)(v >> 32), 63) << 32) | lane_u32((uint32_t)v, 63);
}

// Top-k of the ordered keys keys_lds[0..E), E <= 64 MM, 1 <= k <= min(E, 32):
// larger keys first, equal keys in ascending expert order; sel[0..k) gets the
// experts in that rank order. Lane l holds experts l + 64 m as 64-bit values
// (key << 32 | ~expert) -- larger value = earlier rank, all distinct -- sorted
// descending in registers (odd-even transposition network); each of the k
// rounds takes the wave maximum of the lanes' heads and the winning lane drops
// its head. All in VALU and DPP (no scalar dependency chains). Every lane must
// call it. Returns the k-th largest key.
template <int MM>
__device__ __forceinline__ uint32_t wave_topk_m(const uint32_t *keys_lds, int E, int k, int *sel) {
  const int l = __lane_id();
  uint64_t v[MM];
#pragma unroll
  for (int m = 0; m < MM; ++m) {
    const int e = l + 64 * m;
    v[m] = e < E ? ((uint64_t)keys_lds[e] << 32) | (uint32_t)~e : 0ull;  // real keys are >= 0x007FFFFF
  }
#pragma unroll
  for (int st = 0; st < MM; ++st) {
#pragma unroll
    for (int m = st & 1; m + 1 < MM; m += 2) {
      const uint64_t hi = v[m] > v[m + 1] ? v[m] : v[m + 1];
      const uint64_t lo = v[m] > v[m + 1] ? v[m + 1] : v[m];
      v[m] = hi;
      v[m + 1] = lo;
    }
  }
  uint64_t best = 0;
  for (int r = 0; r < k; ++r) {
    best = wave_max_u64(v[0]);
    const bool win = v[0] == best;
#pragma unroll
    for (int m = 0; m < MM; ++m) v[m] = win ? (m + 1 < MM ? v[m + 1] : 0ull) : v[m];
    if (l == 0) sel[r] = (int)~(uint32_t)best;
  }
  return (uint32_t)(best >> 32);
}

// Value of lane (lane ^ D) for D a power of two below 64: DPP quad permutes
// for 1 and 2, ds_swizzle's xor mode for 4..16 (within 32-lane halves), a
// cross-half shuffle for 32.
template <int D>
__device__ __forceinline__ uint32_t xor_lane(uint32_t v) {
  if constexpr (D == 1) return dpp<kDppQuadXor1, 0xF>(v);
  else if constexpr (D == 2) return dpp<kDppQuadXor2, 0xF>(v);
  else if constexpr (D < 32) return (uint32_t)__builtin_amdgcn_ds_swizzle((int)v, 0x1F | (D << 10));
  else return (uint32_t)__shfl_xor((int)v, 32, kWave);
}

template <int K, int J>
__device__ __forceinline__ uint64_t bitonic_step(uint64_t v, int l) {
  const uint64_t o = ((uint64_t)xor_lane<J>((uint32_t)(v >> 32)) << 32) | xor_lane<J>((uint32_t)v);
  const bool keep_max = ((l & J) == 0) == ((l & K) == 0);
  return keep_max ? (o > v ? o : v) : (o < v ? o : v);
}

template <int K, int J>
__device__ __forceinline__ uint64_t bitonic_merge(uint64_t v, int l) {
  v = bitonic_step<K, J>(v, l);
  if constexpr (J > 1) v = bitonic_merge<K, J / 2>(v, l);
  return v;
}

// Sorts one 64-bit value per lane across the wave, descending (lane 0 holds
// the largest): the 21 compare-exchange stages of a bitonic network.
template <int K = 2>
__device__ __forceinline__ uint64_t wave_sort_desc(uint64_t v) {
  v = bitonic_merge<K, K / 2>(v, __lane_id());
  if constexpr (K < 64) v = wave_sort_desc<K * 2>(v);
  return v;
}

// Top 32 of two lists sorted descending in lanes 0..31 (a and b), sorted
// descending in lanes 0..31: b reversed into lanes 32..63 makes a bitonic
// sequence of 64, which one 6-stage merge sorts.
__device__ __forceinline__ uint64_t merge_top32(uint64_t a, uint64_t b) {
  const int l = __lane_id();
  const uint32_t bl = (uint32_t)__shfl((int)(uint32_t)b, 63 - l, kWave);
  const uint32_t bh = (uint32_t)__shfl((int)(uint32_t)(b >> 32), 63 - l, kWave);
  const uint64_t c = l < 32 ? a : (((uint64_t)bh << 32) | bl);
  return bitonic_merge<64, 32>(c, l);
}

// Inclusive prefix sum over the wave (lane l gets the sum of lanes 0..l):
// DPP shifts inside rows of 16, then the row broadcasts.
__device__ __forceinline__ int wave_incl_scan(int v) {
  v += (int)__builtin_amdgcn_update_dpp(0, v, 0x111, 0xF, 0xF, false);  // row_shr:1
  v += (int)__builtin_amdgcn_update_dpp(0, v, 0x112, 0xF, 0xF, false);  // row_shr:2
  v += (int)__builtin_amdgcn_update_dpp(0, v, 0x114, 0xF, 0xF, false);  // row_shr:4
  v += (int)__builtin_amdgcn_update_dpp(0, v, 0x118, 0xF, 0xF, false);  // row_shr:8
  v += (int)__builtin_amdgcn_update_dpp(0, v, kDppBcast15, 0xA, 0xF, false);
  v += (int)__builtin_amdgcn_update_dpp(0, v, kDppBcast31, 0xC, 0xF, false);
  return v;
}

// Top-k (k <= 32) of up to 64 NG keys by sorting: group g = experts 64 g ..
// 64 g + 63 is sorted across the wave (bitonic network, the NG groups
// independent), then pairs of groups are merged into their 32 best until one
// list remains. Same contract as wave_topk_m.
template <int NG>
__device__ __forceinline__ uint32_t wave_topk_sort(const uint32_t *keys_lds, int E, int k, int *sel) {
  const int l = __lane_id();
  uint64_t v[NG];
#pragma unroll
  for (int g = 0; g < NG; ++g) {
    const int e = 64 * g + l;
    v[g] = e < E ? ((uint64_t)keys_lds[e] << 32) | (uint32_t)~e : 0ull;
  }
#pragma unroll
  for (int g = 0; g < NG; ++g) v[g] = wave_sort_desc(v[g]);
#pragma unroll
  for (int n = NG; n > 1; n /= 2) {
#pragma unroll
    for (int g = 0; g < n / 2; ++g) v[g] = merge_top32(v[2 * g], v[2 * g + 1]);
  }
  if (l < k) sel[l] = (int)~(uint32_t)v[0];
  return lane_u32((uint32_t)(v[0] >> 32), k - 1);
}

__device__ __forceinline__ uint32_t wave_topk(const uint32_t *keys_lds, int E, int k, int *sel) {
  if (E <= 128) return wave_topk_m<2>(keys_lds, E, k, sel);
  if (E <= 256) return wave_topk_m<4>(keys_lds, E, k, sel);
  if (E <= 512) return wave_topk_m<8>(keys_lds, E, k, sel);
  return wave_topk_sort<16>(keys_lds, E, k, sel);  // 16 registers per lane: the sort is 4x faster
}

}  // namespace k3moe
