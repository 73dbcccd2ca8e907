// Shared device helpers for the mHC kernels (gfx950 / CDNA4, wave64).
//
// * storage-type traits: 16-byte vector loads/stores of bf16 / fp16 / fp32
//   rows, converted to and from fp32 registers (round-to-nearest-even on store)
// * wave64 cross-lane reductions
// * bf16 "plane" splitting of fp32 values for exact-enough MFMA contractions
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace mhc {

constexpr int kWave = 64;

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float floatx4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

// ---------------------------------------------------------------------------
// scalar conversions
// ---------------------------------------------------------------------------
__device__ __forceinline__ float bf16_bits_to_f32(uint32_t h) {
  return __uint_as_float(h << 16);
}

typedef float floatx2_t __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));

// fp32 -> bf16 bits, round to nearest even (gfx950 v_cvt_pk_bf16_f32).
__device__ __forceinline__ uint32_t f32_to_bf16_bits(float f) {
  return (uint32_t)__builtin_bit_cast(uint16_t, (__bf16)f);
}

// Two fp32 values -> packed bf16x2 (lo in bits 0..15), one instruction.
__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
  const floatx2_t v = {lo, hi};
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, bf16x2_t));
}

__device__ __forceinline__ float f16_bits_to_f32(uint32_t h) {
  _Float16 v = __builtin_bit_cast(_Float16, (uint16_t)h);
  return (float)v;
}

__device__ __forceinline__ uint32_t f32_to_f16_bits(float f) {
  _Float16 v = (_Float16)f;  // v_cvt_f16_f32, round to nearest even
  return (uint32_t)__builtin_bit_cast(uint16_t, v);
}

// ---------------------------------------------------------------------------
// storage traits.  VEC = elements per 16-byte access.
// ---------------------------------------------------------------------------
struct bf16_t { uint16_t bits; };
struct f16_t { uint16_t bits; };

template <typename S> struct Store;

template <> struct Store<bf16_t> {
  static constexpr int VEC = 8;
  static constexpr int PLANES = 1;  // bf16 planes needed to hold a value exactly
  __device__ static float to_f32(uint16_t b) { return bf16_bits_to_f32(b); }
  __device__ static uint16_t from_f32(float f) { return (uint16_t)f32_to_bf16_bits(f); }
  // 16-byte vector <-> 8 floats
  __device__ static void unpack(const u32x4& v, float* o) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      o[2 * i] = __uint_as_float(v[i] << 16);
      o[2 * i + 1] = __uint_as_float(v[i] & 0xffff0000u);
    }
  }
  __device__ static u32x4 pack(const float* o) {
    u32x4 v;
#pragma unroll
    for (int i = 0; i < 4; ++i) v[i] = pack_bf16x2(o[2 * i], o[2 * i + 1]);
    return v;
  }
};

template <> struct Store<f16_t> {
  static constexpr int VEC = 8;
  static constexpr int PLANES = 2;
  __device__ static float to_f32(uint16_t b) { return f16_bits_to_f32(b); }
  __device__ static uint16_t from_f32(float f) { return (uint16_t)f32_to_f16_bits(f); }
  __device__ static void unpack(const u32x4& v, float* o) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      o[2 * i] = f16_bits_to_f32(v[i] & 0xffffu);
      o[2 * i + 1] = f16_bits_to_f32(v[i] >> 16);
    }
  }
  __device__ static u32x4 pack(const float* o) {
    u32x4 v;
#pragma unroll
    for (int i = 0; i < 4; ++i)
      v[i] = f32_to_f16_bits(o[2 * i]) | (f32_to_f16_bits(o[2 * i + 1]) << 16);
    return v;
  }
};

template <> struct Store<float> {
  static constexpr int VEC = 4;
  static constexpr int PLANES = 2;
  __device__ static void unpack(const u32x4& v, float* o) {
#pragma unroll
    for (int i = 0; i < 4; ++i) o[i] = __uint_as_float(v[i]);
  }
  __device__ static u32x4 pack(const float* o) {
    u32x4 v;
#pragma unroll
    for (int i = 0; i < 4; ++i) v[i] = __float_as_uint(o[i]);
    return v;
  }
};

// Element access used by the unaligned (scalar) paths.
template <typename S> __device__ __forceinline__ float load_elem(const S* p, int64_t i) {
  return Store<S>::to_f32(reinterpret_cast<const uint16_t*>(p)[i]);
}
template <> __device__ __forceinline__ float load_elem<float>(const float* p, int64_t i) {
  return p[i];
}
template <typename S> __device__ __forceinline__ void store_elem(S* p, int64_t i, float v) {
  reinterpret_cast<uint16_t*>(p)[i] = Store<S>::from_f32(v);
}
template <> __device__ __forceinline__ void store_elem<float>(float* p, int64_t i, float v) {
  p[i] = v;
}

__device__ __forceinline__ u32x4 ld16(const void* p) {
  return *reinterpret_cast<const u32x4*>(p);
}
__device__ __forceinline__ void st16(void* p, const u32x4& v) {
  *reinterpret_cast<u32x4*>(p) = v;
}
// 16-byte load that bypasses cache retention (data read exactly once).
__device__ __forceinline__ u32x4 ld16nt(const void* p) {
  return __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p));
}
// 16-byte streaming store (output not re-read by this kernel).
__device__ __forceinline__ void st16nt(void* p, const u32x4& v) {
  __builtin_nontemporal_store(v, reinterpret_cast<u32x4*>(p));
}

// ---------------------------------------------------------------------------
// XCD-contiguous work order.  Workgroups are dispatched round robin over the
// eight XCDs (workgroup b runs on XCD b % 8); xcd_contig maps b to an item so
// that each XCD walks one contiguous eighth of the nb items in order (XCD x
// gets items [x * q + min(x, r), ..) with q = nb / 8, r = nb % 8; a bijection
// on [0, nb)).  Token-streaming kernels read each XCD's rows as long runs
// this way instead of interleaving all eight XCDs over every stretch of
// memory.  Which kernels gain is measured, not predictable: on the MI355X
// the N = 4 post forward (c5 1446 -> 1360 us) and the N = 8 wave-per-token
// post backward (config 4 670-730 -> 602-617 us) do; the N = 8 post forward,
// the post backward's block kernel, the persistent LDS-pipelined post
// kernels, the pre forward's y pass and the pre backward's kernel A measured
// equal or slower and keep the plain order.
// ---------------------------------------------------------------------------
constexpr int kXcds = 8;
__device__ __forceinline__ int64_t xcd_contig(int64_t b, int64_t nb) {
  const int64_t q = nb / kXcds, r = nb % kXcds, x = b % kXcds;
  return x * q + (x < r ? x : r) + b / kXcds;
}

// ---------------------------------------------------------------------------
// wave64 reductions
// ---------------------------------------------------------------------------
__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) v += __shfl_xor(v, o, kWave);
  return v;
}

// DPP lane moves inside 16-lane rows (a few cycles, no LDS round trip):
// quad_perm swaps lanes xor 1 / xor 2, row_ror rotates a row by 4 / 8 lanes
// (row_ror:8 is lane xor 8).
template <int CTRL>
__device__ __forceinline__ float dpp_mov(float v) {
  return __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), CTRL, 0xF, 0xF, false));
}
constexpr int kDppXor1 = 0xB1;  // quad_perm [1,0,3,2]
constexpr int kDppXor2 = 0x4E;  // quad_perm [2,3,0,1]
constexpr int kDppRor4 = 0x124;
constexpr int kDppRor8 = 0x128;
constexpr int kDppHalfMirror = 0x141;  // row_half_mirror: lane l <- 7 - l within each 8 lanes

// v + (v of lane xor 16) and v + (v of lane xor 32) with the gfx950 lane
// swaps (one VALU instruction, no LDS round trip).  permlane16_swap(a, b)
// exchanges the odd 16-lane rows of a with the even rows of b, permlane32
// the upper half of a with the lower half of b; with a = b = v the two
// results hold, lane for lane, v and its partner's v (in some order), so
// their sum is the pair sum.
__device__ __forceinline__ float add_xor16(float v) {
  const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}
__device__ __forceinline__ float add_xor32(float v) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}
__device__ __forceinline__ float max_xor16(float v) {
  const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float max_xor32(float v) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}

// Sum over lanes whose indices differ only in the bits of `mask`
// (mask is a compile-time set of xor offsets, e.g. 0b0011 -> offsets 1 and 2).
// Offsets 1, 2, 8 and the pair {4, 8} run on DPP, 4 after 1 and 2 as a
// half-row mirror (every lane of a quad then holds the quad's sum), 16 and
// 32 on the lane swaps; only 4 alone is a cross-lane shuffle.  Each step
// adds a lane's value to its partner's, so the bits equal those of the
// __shfl_xor form.
template <int MASK>
__device__ __forceinline__ float group_sum(float v) {
  if constexpr (MASK & 1) v += dpp_mov<kDppXor1>(v);
  if constexpr (MASK & 2) v += dpp_mov<kDppXor2>(v);
  if constexpr ((MASK & 12) == 12) {
    v += dpp_mov<kDppRor4>(v);  // {l, l-4}
    v += dpp_mov<kDppRor8>(v);  // {l, l-4, l-8, l-12}: the 4 lanes of l's class mod 4
  } else if constexpr (MASK & 8) {
    v += dpp_mov<kDppRor8>(v);
  } else if constexpr ((MASK & 7) == 7) {
    v += dpp_mov<kDppHalfMirror>(v);  // the other quad of the 8 lanes
  } else if constexpr (MASK & 4) {
    v += __shfl_xor(v, 4, kWave);
  }
  if constexpr (MASK & 16) v = add_xor16(v);
  if constexpr (MASK & 32) v = add_xor32(v);
  return v;
}
// Sums each of R values (R % 4 == 0) over the 64 lanes of the wave with two
// values per lane swap on the xor-32 and xor-16 levels: v_permlane32_swap
// exchanges lanes 32..63 of its first operand with lanes 0..31 of its
// second (v_permlane16_swap the odd 16-lane rows of the first with the even
// rows of the second), so one swap and one add combine two values, halving
// the registers each level; then DPP adds within each 16-lane row.
// Afterwards every lane of row rho (lanes 16rho..16rho+15) of v[k], k < R/4,
// holds the total of value k + rho * R / 4.  2.5 R VALU instructions against
// 8 R for group_sum<63> on each value (12 R and 6 R LDS swizzles for
// wave_sum).
template <int R>
__device__ __forceinline__ void wave_sum_rows(float (&v)[R]) {
  static_assert(R % 4 == 0, "four rows of R / 4 values");
  constexpr int H = R / 2, Q = R / 4;
#pragma unroll
  for (int k = 0; k < H; ++k) {  // v[k]: value k in lanes 0..31, value k + H in 32..63
    const auto s = __builtin_amdgcn_permlane32_swap(__float_as_uint(v[k]), __float_as_uint(v[k + H]), false, false);
    v[k] = __uint_as_float(s[0]) + __uint_as_float(s[1]);
  }
#pragma unroll
  for (int k = 0; k < Q; ++k) {  // v[k]: rows 0..3 hold values k, k + Q, k + H, k + H + Q
    const auto s = __builtin_amdgcn_permlane16_swap(__float_as_uint(v[k]), __float_as_uint(v[k + Q]), false, false);
    v[k] = __uint_as_float(s[0]) + __uint_as_float(s[1]);
  }
#pragma unroll
  for (int k = 0; k < Q; ++k) v[k] = group_sum<15>(v[k]);
}

template <int MASK>
__device__ __forceinline__ float group_max(float v) {
  if constexpr (MASK & 1) v = fmaxf(v, dpp_mov<kDppXor1>(v));
  if constexpr (MASK & 2) v = fmaxf(v, dpp_mov<kDppXor2>(v));
  if constexpr ((MASK & 12) == 12) {
    v = fmaxf(v, dpp_mov<kDppRor4>(v));
    v = fmaxf(v, dpp_mov<kDppRor8>(v));
  } else if constexpr (MASK & 8) {
    v = fmaxf(v, dpp_mov<kDppRor8>(v));
  } else if constexpr ((MASK & 7) == 7) {
    v = fmaxf(v, dpp_mov<kDppHalfMirror>(v));
  } else if constexpr (MASK & 4) {
    v = fmaxf(v, __shfl_xor(v, 4, kWave));
  }
  if constexpr (MASK & 16) v = max_xor16(v);
  if constexpr (MASK & 32) v = max_xor32(v);
  return v;
}

// ---------------------------------------------------------------------------
// bf16 planes: v ~= p0 + p1 (+ p2), each a bf16 (returned as raw bits).
// Two planes leave a relative residual below 2^-17; fp16 inputs are exact.
// ---------------------------------------------------------------------------
__device__ __forceinline__ void split2_bf16(float v, uint32_t& hi, uint32_t& lo) {
  hi = f32_to_bf16_bits(v);
  float r = v - bf16_bits_to_f32(hi);
  lo = f32_to_bf16_bits(r);
}

}  // namespace mhc
