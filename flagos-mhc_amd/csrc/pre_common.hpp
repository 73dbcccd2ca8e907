// Helpers shared by the mhc_pre_clamp_sinkhorn forward and backward kernels:
// problem dimensions, MFMA wrapper and the conversion of 8-element groups of
// activations into bf16 "planes" (MFMA operands whose sum reproduces the
// value: 1 plane for bf16, 2 for fp16 (exact), 3 for fp32 (2^-26 relative)).
#pragma once

#include "common.hpp"
#include "lds_dma.hpp"

namespace mhc {

template <int N> struct PreDims {
  static constexpr int M = 2 * N + N * N;     // hcMix
  static constexpr int MT = (M + 15) / 16;    // 16-row m tiles
  static constexpr int MP = MT * 16;          // m padded to 16
  static constexpr int MK = (M + 31) / 32;    // 32-deep m chunks (MFMA K)
  static constexpr int MP32 = MK * 32;        // m padded to 32
};

__device__ __forceinline__ floatx4 mfma16x16x32(const bf16x8& a, const bf16x8& b, floatx4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}

__device__ __forceinline__ bf16x8 as_bf16x8(const u32x4& v) { return __builtin_bit_cast(bf16x8, v); }

__device__ __forceinline__ u32x4 zero4() {
  u32x4 z;
  z[0] = z[1] = z[2] = z[3] = 0u;
  return z;
}

// Split 8 fp32 values into three bf16 planes (hi, mid, lo): residual below
// 2^-26 relative.
__device__ __forceinline__ void split8x3(const float* f, u32x4& p0, u32x4& p1, u32x4& p2) {
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    uint32_t h[2], m[2], l[2];
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      float v = f[2 * i + j];
      h[j] = f32_to_bf16_bits(v);
      v -= bf16_bits_to_f32(h[j]);
      m[j] = f32_to_bf16_bits(v);
      v -= bf16_bits_to_f32(m[j]);
      l[j] = f32_to_bf16_bits(v);
    }
    p0[i] = h[0] | (h[1] << 16);
    p1[i] = m[0] | (m[1] << 16);
    p2[i] = l[0] | (l[1] << 16);
  }
}

// Split 8 fp32 values into two bf16 planes (hi, lo), packed as bf16x8.
__device__ __forceinline__ void split8(const float* f, u32x4& hi, u32x4& lo) {
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    uint32_t h0, l0, h1, l1;
    split2_bf16(f[2 * i], h0, l0);
    split2_bf16(f[2 * i + 1], h1, l1);
    hi[i] = h0 | (h1 << 16);
    lo[i] = l0 | (l1 << 16);
  }
}

// Branch-free masked 16-byte load of p[k..k+8): the address is clamped into
// [0, lim) (lim >= 8, lim % 8 == 0) and the result zeroed when !(ok && k < lim),
// so the load issues unconditionally and never leaves the row.  `p` must be a
// valid row even when !ok.
__device__ __forceinline__ u32x4 ld16_masked(const void* p, int64_t k, int64_t lim, bool ok,
                                             int elem_bytes) {
  const int64_t kk = k < lim ? k : lim - 8;
  u32x4 v = ld16nt(static_cast<const char*>(p) + kk * elem_bytes);
  return (ok && k < lim) ? v : zero4();
}

// Group of 8 consecutive activations [k, k+8) of a row holding `lim` valid
// elements.  VEC: the row is 16-byte aligned and lim % 8 == 0 (whole group in
// or out); otherwise elements are loaded one by one with bounds checks.
// On the VEC path `row` must point at a valid row even when !ok.
template <typename S> struct XGroup;

template <> struct XGroup<bf16_t> {
  static constexpr int PLANES = 1;
  template <bool VEC>
  __device__ static void load(const bf16_t* row, int64_t k, int64_t lim, bool ok, u32x4 (&pl)[1],
                              float* f) {
    u32x4 v = zero4();
    if constexpr (VEC) {
      v = ld16_masked(row, k, lim, ok, 2);
    } else {
      const uint16_t* r = reinterpret_cast<const uint16_t*>(row);
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        uint32_t a = (ok && k + 2 * i < lim) ? r[k + 2 * i] : 0u;
        uint32_t b = (ok && k + 2 * i + 1 < lim) ? r[k + 2 * i + 1] : 0u;
        v[i] = a | (b << 16);
      }
    }
    pl[0] = v;
    Store<bf16_t>::unpack(v, f);
  }
};

template <> struct XGroup<f16_t> {
  static constexpr int PLANES = 2;
  template <bool VEC>
  __device__ static void load(const f16_t* row, int64_t k, int64_t lim, bool ok, u32x4 (&pl)[2],
                              float* f) {
    if constexpr (VEC) {
      Store<f16_t>::unpack(ld16_masked(row, k, lim, ok, 2), f);
    } else {
#pragma unroll
      for (int i = 0; i < 8; ++i) f[i] = (ok && k + i < lim) ? load_elem(row, k + i) : 0.f;
    }
    split8(f, pl[0], pl[1]);
  }
};

template <> struct XGroup<float> {
  static constexpr int PLANES = 3;
  template <bool VEC>
  __device__ static void load(const float* row, int64_t k, int64_t lim, bool ok, u32x4 (&pl)[3],
                              float* f) {
    if constexpr (VEC) {
      const u32x4 a = ld16_masked(row, k, lim, ok, 4), b = ld16_masked(row + 4, k, lim, ok, 4);
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        f[i] = __uint_as_float(a[i]);
        f[4 + i] = __uint_as_float(b[i]);
      }
    } else {
#pragma unroll
      for (int i = 0; i < 8; ++i) f[i] = (ok && k + i < lim) ? row[k + i] : 0.f;
    }
    split8x3(f, pl[0], pl[1], pl[2]);
  }
};

// Store 8 consecutive fp32 values as storage type S at p[k..k+8) (VEC:
// 16B-aligned, stored only if the whole group lies below `lim`) or element
// by element up to `lim`.
template <typename S, bool VEC>
__device__ __forceinline__ void store8(S* p, int64_t k, int64_t lim, const float* f) {
  if constexpr (VEC) {
    if (k + 8 > lim) return;
    if constexpr (sizeof(S) == 2) {
      st16(p + k, Store<S>::pack(f));
    } else {
      st16(p + k, Store<float>::pack(f));
      st16(p + k + 4, Store<float>::pack(f + 4));
    }
  } else {
#pragma unroll
    for (int i = 0; i < 8; ++i)
      if (k + i < lim) store_elem(p, k + i, f[i]);
  }
}

// Load 8 consecutive values as fp32 (VEC / scalar as above), streamed past
// the caches.  On the VEC path the load is branch-free and `p` must be a
// valid row even when !ok.
template <typename S, bool VEC>
__device__ __forceinline__ void load8f(const S* p, int64_t k, int64_t lim, bool ok, float* f) {
  if constexpr (VEC) {
    if constexpr (sizeof(S) == 2) {
      Store<S>::unpack(ld16_masked(p, k, lim, ok, 2), f);
    } else {
      Store<float>::unpack(ld16_masked(p, k, lim, ok, 4), f);
      Store<float>::unpack(ld16_masked(p + 4, k, lim, ok, 4), f + 4);
    }
  } else {
#pragma unroll
    for (int i = 0; i < 8; ++i) f[i] = (ok && k + i < lim) ? load_elem(p, k + i) : 0.f;
  }
}

}  // namespace mhc
