// Shared device/host helpers for the gfx950 weight-only quantized Linear kernels.
//
// Conventions used by every kernel in this library:
//   * activations x and outputs y are bf16, row-major with an explicit row stride (elements);
//   * packed weights are byte arrays with an explicit row stride (bytes);
//   * scale / zero carry (n, g) strides in elements and a dtype code (IMQ_DT_*);
//   * every launch goes to the caller's stream; no kernel allocates, frees or synchronizes.
#pragma once

#include <hip/hip_runtime.h>
#include <hip/hip_bf16.h>
#include <hip/hip_fp16.h>
#include <stdint.h>

#include "../../include/imq.h"

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));
typedef float f32x16_t __attribute__((ext_vector_type(16)));
typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2_t __attribute__((ext_vector_type(2)));

#define IMQ_DEV __device__ __forceinline__
#define IMQ_HOST_DEV __host__ __device__

// ---- bf16 / fp16 <-> fp32 (bit-level, round-to-nearest-even) --------------------------------
IMQ_DEV float bf16_bits_to_f32(uint32_t b) { return __uint_as_float(b << 16); }

IMQ_DEV uint32_t f32_to_bf16_bits(float f) {
  // RNE; NaN kept quiet. Same rule as torch's float -> bfloat16 conversion.
  uint32_t u = __float_as_uint(f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return 0x7fc0u;
  return (u + 0x7fffu + ((u >> 16) & 1u)) >> 16;
}

IMQ_DEV float round_bf16(float f) { return __uint_as_float(f32_to_bf16_bits(f) << 16); }

// fp16 <-> fp32 through _Float16 bit casts (v_cvt_f32_f16 / v_cvt_f16_f32, round to nearest even);
// the __half helpers go through a union that can leave a stack slot behind in unrolled code.
IMQ_DEV float f16_bits_to_f32(uint32_t b) { return (float)__builtin_bit_cast(_Float16, (uint16_t)b); }
IMQ_DEV uint32_t f32_to_f16_bits(float f) { return __builtin_bit_cast(uint16_t, (_Float16)f); }

IMQ_DEV float round_fp16(float f) { return (float)(_Float16)f; }

// Load element `idx` of a dtype-coded array as fp32 (exact widening).
template <int DT>
IMQ_DEV float load_as_f32(const void* p, int64_t idx) {
  if constexpr (DT == IMQ_DT_BF16) {
    return bf16_bits_to_f32(((const uint16_t*)p)[idx]);
  } else if constexpr (DT == IMQ_DT_FP16) {
    return f16_bits_to_f32(((const uint16_t*)p)[idx]);
  } else {
    return ((const float*)p)[idx];
  }
}

// Raw bits of element `idx` (16-bit dtypes zero-extended); raw_bits_to_f32 widens them. Loading
// raw bits lets a kernel keep the load in flight and convert only where the value is consumed.
template <int DT>
IMQ_DEV uint32_t load_raw_bits(const void* p, int64_t idx) {
  if constexpr (DT == IMQ_DT_FP32) return ((const uint32_t*)p)[idx];
  else return ((const uint16_t*)p)[idx];
}

template <int DT>
IMQ_DEV float raw_bits_to_f32(uint32_t b) {
  if constexpr (DT == IMQ_DT_BF16) return __uint_as_float(b << 16);
  else if constexpr (DT == IMQ_DT_FP16) return f16_bits_to_f32(b);
  else return __uint_as_float(b);
}

// Round an fp32 value to dtype DT (result kept as fp32).
template <int DT>
IMQ_DEV float round_to(float f) {
  if constexpr (DT == IMQ_DT_BF16) return round_bf16(f);
  else if constexpr (DT == IMQ_DT_FP16) return round_fp16(f);
  else return f;
}

// Load a scale/zero element and round it to bf16, i.e. `t.to(torch.bfloat16)` of the stored
// value -- the operand the reference dequant `_dequant(torch.bfloat16)` multiplies with.
template <int DT>
IMQ_DEV float load_as_bf16_f32(const void* p, int64_t idx) {
  float v = load_as_f32<DT>(p, idx);
  if constexpr (DT == IMQ_DT_BF16) return v;
  else return round_bf16(v);
}

template <int DT>
IMQ_DEV void store_from_f32(void* p, int64_t idx, float v) {
  if constexpr (DT == IMQ_DT_BF16) {
    ((uint16_t*)p)[idx] = (uint16_t)f32_to_bf16_bits(v);
  } else if constexpr (DT == IMQ_DT_FP16) {
    ((uint16_t*)p)[idx] = (uint16_t)f32_to_f16_bits(v);
  } else {
    ((float*)p)[idx] = v;
  }
}

// Two fp32 values -> packed bf16x2 (lo in bits 0..15), round-to-nearest-even: one
// v_cvt_pk_bf16_f32 on gfx950. Same results as f32_to_bf16_bits for every non-NaN input.
typedef float f32x2_t __attribute__((ext_vector_type(2)));
IMQ_DEV uint32_t cvt_pk_bf16(float lo, float hi) {
  const f32x2_t v = {lo, hi};
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, bf16x2_t));
}

// fp32 -> nearest bf16 (ties to even), kept as fp32: one v_cvt_pk_bf16_f32 and a shift. Equal
// to round_bf16 for every finite input.
IMQ_DEV float round_bf16_hw(float f) { return __uint_as_float(cvt_pk_bf16(f, 0.f) << 16); }

// Raw 16/32-bit scale/zero bits -> fp32 value rounded to bf16 (the operand of the reference
// dequant `_dequant(torch.bfloat16)`), converted where it is consumed.
template <int DT>
IMQ_DEV float raw_to_bf16_f32(uint32_t r) {
  if constexpr (DT == IMQ_DT_BF16) return __uint_as_float(r << 16);
  else if constexpr (DT == IMQ_DT_FP16) return round_bf16_hw(f16_bits_to_f32(r));
  else return round_bf16_hw(__uint_as_float(r));
}

// (a & m) | o  -> v_and_or_b32
IMQ_DEV uint32_t and_or(uint32_t a, uint32_t m, uint32_t o) { return (a & m) | o; }

IMQ_DEV uint32_t perm_b32(uint32_t hi, uint32_t lo, uint32_t sel) {
  return __builtin_amdgcn_perm(hi, lo, sel);
}

// The bf16 bit pattern 0x4300 (= 128.0) in both halves, produced in a VGPR the compiler cannot
// constant-fold: `(x & mask) | magic` then selects one v_and_or_b32 (mask in an SGPR, magic in
// a VGPR), since a gfx9-family VOP3 cannot encode the two literals. The unpack itself stays
// plain C so the compiler sees every VALU write that feeds an MFMA operand and inserts the
// required wait states (an inline-asm VALU op is invisible to its hazard recognizer).
IMQ_DEV uint32_t magic_bf16_128x2() {
  uint32_t r;
  asm volatile("v_mov_b32 %0, 0x43004300" : "=v"(r));
  return r;
}

// 8 int4 codes (one u32, code i at bits 4i..4i+3) -> 8 bf16 values (128 + code), exact:
// (code | 0x4300) is the bf16 128 + code. Seven VALU ops for eight weights.
// Output element order is [c0, c4, c1, c5, c2, c6, c3, c7]; activations fed against these
// operands must use the same order (see permute_x8).
IMQ_DEV bf16x8_t unpack_nib8_bf16(uint32_t w, uint32_t magic) {
  u32x4_t r;
  r[0] = (w & 0x000F000Fu) | magic;
  r[1] = ((w >> 4) & 0x000F000Fu) | magic;
  r[2] = ((w >> 8) & 0x000F000Fu) | magic;
  r[3] = ((w >> 12) & 0x000F000Fu) | magic;
  return __builtin_bit_cast(bf16x8_t, r);
}

// 8 consecutive bf16 activations (16 bytes as 4 dwords) -> order [x0,x4,x1,x5,x2,x6,x3,x7].
IMQ_DEV u32x4_t permute_x8(u32x4_t v) {
  u32x4_t p;
  p[0] = perm_b32(v[2], v[0], 0x05040100u);
  p[1] = perm_b32(v[2], v[0], 0x07060302u);
  p[2] = perm_b32(v[3], v[1], 0x05040100u);
  p[3] = perm_b32(v[3], v[1], 0x07060302u);
  return p;
}

// Lane c of each 16-lane row receives lane (c - N) & 15 of the same row (DPP row_ror:N): a VALU
// operand modifier instead of an LDS permute with its address arithmetic and round trip.
template <int N>
IMQ_DEV uint32_t dpp_row_ror(uint32_t v) {
  return (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x120 + N, 0xf, 0xf, false);
}
template <int N>
IMQ_DEV float dpp_row_ror(float v) { return __uint_as_float(dpp_row_ror<N>(__float_as_uint(v))); }

// Sum over the 16 lanes of each row, returned to every lane. After the n-th step the values
// repeat with period 16 >> n, so rotations by 8, 4, 2, 1 reach the same partner values as the
// xor butterfly (`v += __shfl_xor(v, 8 / 4 / 2 / 1, 16)`) and give the same bits.
IMQ_DEV float row_sum16(float v) {
  v += dpp_row_ror<8>(v);
  v += dpp_row_ror<4>(v);
  v += dpp_row_ror<2>(v);
  v += dpp_row_ror<1>(v);
  return v;
}

// Sum over each group of 4 lanes (DPP quad_perm [1,0,3,2] then [2,3,0,1]): the xor-1 / xor-2
// butterfly exactly.
IMQ_DEV float quad_sum4(float v) {
  v += __uint_as_float((uint32_t)__builtin_amdgcn_update_dpp(0, (int)__float_as_uint(v), 0xB1, 0xf, 0xf, false));
  v += __uint_as_float((uint32_t)__builtin_amdgcn_update_dpp(0, (int)__float_as_uint(v), 0x4E, 0xf, 0xf, false));
  return v;
}

// Sum over each group of 8 lanes: the quad sums, then the other quad's through row_half_mirror
// (lane c of 8 reads lane 7 - c, which holds the other quad's sum).
IMQ_DEV float half_row_sum8(float v) {
  v = quad_sum4(v);
  v += __uint_as_float((uint32_t)__builtin_amdgcn_update_dpp(0, (int)__float_as_uint(v), 0x141, 0xf, 0xf, false));
  return v;
}

// Sum of the 8 bf16 values of a 16-byte block: four v_dot2c_f32_bf16 against (1, 1), one VALU
// operation per two values (instead of two conversions and two adds).
IMQ_DEV float bf16x8_sum(u32x4_t v) {
  const bf16x2_t one = __builtin_bit_cast(bf16x2_t, 0x3f803f80u);
  float s = 0.f;
#pragma unroll
  for (int d = 0; d < 4; ++d) {
    // the element goes through a scalar first: hipcc bit-casts a subscripted vector element
    // `v[d]` from element 0 whatever d is
    const uint32_t w = v[d];
    s = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, w), one, s, false);
  }
  return s;
}

// 32x32x16 bf16: A lane l = row l%32, K 8*(l/32)..+8; B lane l = column l%32, same K; D lane l
// holds column l%32, element r at row 8*(r/4) + 4*(l/32) + r%4. Twice the 16x16x32 rate.
IMQ_DEV f32x16_t mfma32x32x16(bf16x8_t a, bf16x8_t b, f32x16_t c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
}

IMQ_DEV f32x4_t mfma16x16x32(bf16x8_t a, bf16x8_t b, f32x4_t c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}

// Workgroup barrier that orders LDS only. __syncthreads() also waits for every outstanding
// global load (vmcnt(0)), which would drain the prefetched weight stream at each barrier.
IMQ_DEV void lds_barrier() { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); }

static inline int64_t imq_cdiv(int64_t a, int64_t b) { return (a + b - 1) / b; }

// Host-side launch error check: hipGetLastError after a launch, mapped to an int status.
#define IMQ_LAUNCH_CHECK()                                   \
  do {                                                       \
    hipError_t _e = hipGetLastError();                       \
    if (_e != hipSuccess) return (int)_e;                    \
  } while (0)

// Per-device attributes the launchers size grids and LDS with (read once per device).
struct DevInfo {
  int cus;
  int max_lds;
};

inline DevInfo device_info() {
  static DevInfo cache[64];
  static int ready[64];
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return DevInfo{256, 65536};
  if (!__atomic_load_n(&ready[dev], __ATOMIC_ACQUIRE)) {
    DevInfo d{256, 65536};
    int v = 0;
    if (hipDeviceGetAttribute(&v, hipDeviceAttributeMultiprocessorCount, dev) == hipSuccess && v > 0)
      d.cus = v;
    if (hipDeviceGetAttribute(&v, hipDeviceAttributeMaxSharedMemoryPerBlock, dev) == hipSuccess && v > 0)
      d.max_lds = v;
    cache[dev] = d;
    __atomic_store_n(&ready[dev], 1, __ATOMIC_RELEASE);
  }
  return cache[dev];
}
