// mhc_post forward and backward: one wave64 per token, streaming over D.
//
//   y[t,i,:]      = sum_j h_res[t,j,i] * x[t,j,:] + h_post[t,i] * h_out[t,:]
//   grad_x[t,j,:] = sum_i h_res[t,j,i] * gy[t,i,:]
//   grad_h_out    = sum_i h_post[t,i] * gy[t,i,:]
//   grad_h_res[t,j,i] = <x[t,j,:], gy[t,i,:]>,  grad_h_post[t,i] = <h_out[t,:], gy[t,i,:]>
//
// Semantics follow the reference's mhc_post_ref / mhc_post_backward_ref
// (src/mhc_post.py:344-352, src/mhc_post_backward.py:624-643).
//
// Layout: x, y, gy, grad_x are contiguous (T, N, D); h_out / grad_h_out are
// (T, D); gates are fp32 (T, N, N) and (T, N).  A wave owns one token: the
// N*N + N gates are wave-uniform scalar loads, every lane streams 16-byte
// vectors of each of the N rows, accumulates in fp32 and stores with
// round-to-nearest-even (streaming stores: outputs are not re-read here).
// The backward's N*N + N dot products are reduced across the wave once per
// token and written by plain stores (no atomics), so results are
// deterministic.
#include "common.hpp"
#include "mhc_launch.hpp"

namespace mhc {

constexpr int kPostWavesPerBlock = 4;

template <int N, typename S, bool VECTOR>
__global__ __launch_bounds__(256) void post_fwd_kernel(
    const S* __restrict__ x, const float* __restrict__ h_res, const S* __restrict__ h_out,
    const float* __restrict__ h_post, S* __restrict__ y, int64_t T, int D) {
  const int lane = threadIdx.x & (kWave - 1);
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int64_t t = (int64_t)blockIdx.x * kPostWavesPerBlock + wave;
  if (t >= T) return;

  float hr[N * N], hp[N];
#pragma unroll
  for (int i = 0; i < N * N; ++i) hr[i] = h_res[t * (N * N) + i];
#pragma unroll
  for (int i = 0; i < N; ++i) hp[i] = h_post[t * N + i];

  const int64_t xrow = t * (int64_t)N * D;
  const int64_t hrow = t * (int64_t)D;

  if constexpr (VECTOR) {
    constexpr int V = Store<S>::VEC;
#pragma unroll 2
    for (int d = lane * V; d < D; d += kWave * V) {
      float xv[N][V], hv[V];
#pragma unroll
      for (int j = 0; j < N; ++j) Store<S>::unpack(ld16(x + xrow + (int64_t)j * D + d), xv[j]);
      Store<S>::unpack(ld16(h_out + hrow + d), hv);
#pragma unroll
      for (int i = 0; i < N; ++i) {
        float o[V];
#pragma unroll
        for (int e = 0; e < V; ++e) {
          float acc = hp[i] * hv[e];
#pragma unroll
          for (int j = 0; j < N; ++j) acc = fmaf(hr[j * N + i], xv[j][e], acc);
          o[e] = acc;
        }
        st16nt(y + xrow + (int64_t)i * D + d, Store<S>::pack(o));
      }
    }
  } else {
    for (int d = lane; d < D; d += kWave) {
      float xv[N];
#pragma unroll
      for (int j = 0; j < N; ++j) xv[j] = load_elem(x, xrow + (int64_t)j * D + d);
      const float hv = load_elem(h_out, hrow + d);
#pragma unroll
      for (int i = 0; i < N; ++i) {
        float acc = hp[i] * hv;
#pragma unroll
        for (int j = 0; j < N; ++j) acc = fmaf(hr[j * N + i], xv[j], acc);
        store_elem(y, xrow + (int64_t)i * D + d, acc);
      }
    }
  }
}

template <int N, typename S, bool VECTOR>
__global__ __launch_bounds__(256) void post_bwd_kernel(
    const S* __restrict__ gy, const S* __restrict__ x, const float* __restrict__ h_res,
    const S* __restrict__ h_out, const float* __restrict__ h_post, S* __restrict__ gx,
    float* __restrict__ g_hres, S* __restrict__ g_hout, float* __restrict__ g_hpost,
    int64_t T, int D) {
  const int lane = threadIdx.x & (kWave - 1);
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int64_t t = (int64_t)blockIdx.x * kPostWavesPerBlock + wave;
  if (t >= T) return;

  float hr[N * N], hp[N];
#pragma unroll
  for (int i = 0; i < N * N; ++i) hr[i] = h_res[t * (N * N) + i];
#pragma unroll
  for (int i = 0; i < N; ++i) hp[i] = h_post[t * N + i];

  float acc_r[N * N], acc_p[N];
#pragma unroll
  for (int i = 0; i < N * N; ++i) acc_r[i] = 0.f;
#pragma unroll
  for (int i = 0; i < N; ++i) acc_p[i] = 0.f;

  const int64_t xrow = t * (int64_t)N * D;
  const int64_t hrow = t * (int64_t)D;

  if constexpr (VECTOR) {
    constexpr int V = Store<S>::VEC;
    for (int d = lane * V; d < D; d += kWave * V) {
      float gv[N][V], xv[N][V], hv[V];
#pragma unroll
      for (int i = 0; i < N; ++i) Store<S>::unpack(ld16(gy + xrow + (int64_t)i * D + d), gv[i]);
#pragma unroll
      for (int j = 0; j < N; ++j) Store<S>::unpack(ld16(x + xrow + (int64_t)j * D + d), xv[j]);
      Store<S>::unpack(ld16(h_out + hrow + d), hv);
#pragma unroll
      for (int j = 0; j < N; ++j) {
        float o[V];
#pragma unroll
        for (int e = 0; e < V; ++e) {
          float a = 0.f;
#pragma unroll
          for (int i = 0; i < N; ++i) a = fmaf(hr[j * N + i], gv[i][e], a);
          o[e] = a;
        }
        st16nt(gx + xrow + (int64_t)j * D + d, Store<S>::pack(o));
      }
      float oh[V];
#pragma unroll
      for (int e = 0; e < V; ++e) {
        float a = 0.f;
#pragma unroll
        for (int i = 0; i < N; ++i) a = fmaf(hp[i], gv[i][e], a);
        oh[e] = a;
      }
      st16nt(g_hout + hrow + d, Store<S>::pack(oh));
#pragma unroll
      for (int e = 0; e < V; ++e) {
#pragma unroll
        for (int j = 0; j < N; ++j)
#pragma unroll
          for (int i = 0; i < N; ++i) acc_r[j * N + i] = fmaf(xv[j][e], gv[i][e], acc_r[j * N + i]);
#pragma unroll
        for (int i = 0; i < N; ++i) acc_p[i] = fmaf(hv[e], gv[i][e], acc_p[i]);
      }
    }
  } else {
    for (int d = lane; d < D; d += kWave) {
      float gv[N], xv[N];
#pragma unroll
      for (int i = 0; i < N; ++i) gv[i] = load_elem(gy, xrow + (int64_t)i * D + d);
#pragma unroll
      for (int j = 0; j < N; ++j) xv[j] = load_elem(x, xrow + (int64_t)j * D + d);
      const float hv = load_elem(h_out, hrow + d);
#pragma unroll
      for (int j = 0; j < N; ++j) {
        float a = 0.f;
#pragma unroll
        for (int i = 0; i < N; ++i) a = fmaf(hr[j * N + i], gv[i], a);
        store_elem(gx, xrow + (int64_t)j * D + d, a);
      }
      float a = 0.f;
#pragma unroll
      for (int i = 0; i < N; ++i) a = fmaf(hp[i], gv[i], a);
      store_elem(g_hout, hrow + d, a);
#pragma unroll
      for (int j = 0; j < N; ++j)
#pragma unroll
        for (int i = 0; i < N; ++i) acc_r[j * N + i] = fmaf(xv[j], gv[i], acc_r[j * N + i]);
#pragma unroll
      for (int i = 0; i < N; ++i) acc_p[i] = fmaf(hv, gv[i], acc_p[i]);
    }
  }

#pragma unroll
  for (int i = 0; i < N * N; ++i) acc_r[i] = wave_sum(acc_r[i]);
#pragma unroll
  for (int i = 0; i < N; ++i) acc_p[i] = wave_sum(acc_p[i]);
  if (lane == 0) {
#pragma unroll
    for (int i = 0; i < N * N; ++i) g_hres[t * (N * N) + i] = acc_r[i];
#pragma unroll
    for (int i = 0; i < N; ++i) g_hpost[t * N + i] = acc_p[i];
  }
}

// ---------------------------------------------------------------------------
// host launchers
// ---------------------------------------------------------------------------
template <int N, typename S>
static int launch_post_fwd(const void* x, const float* h_res, const void* h_out,
                           const float* h_post, void* y, int64_t T, int D, hipStream_t st) {
  const dim3 grid((unsigned)((T + kPostWavesPerBlock - 1) / kPostWavesPerBlock));
  const dim3 block(kWave * kPostWavesPerBlock);
  const bool vec = (D % Store<S>::VEC == 0) && aligned16(x) && aligned16(h_out) && aligned16(y);
  if (vec)
    hipLaunchKernelGGL((post_fwd_kernel<N, S, true>), grid, block, 0, st, (const S*)x, h_res,
                       (const S*)h_out, h_post, (S*)y, T, D);
  else
    hipLaunchKernelGGL((post_fwd_kernel<N, S, false>), grid, block, 0, st, (const S*)x, h_res,
                       (const S*)h_out, h_post, (S*)y, T, D);
  return check_launch("post_fwd");
}

template <int N, typename S>
static int launch_post_bwd(const void* gy, const void* x, const float* h_res, const void* h_out,
                           const float* h_post, void* gx, float* g_hres, void* g_hout,
                           float* g_hpost, int64_t T, int D, hipStream_t st) {
  const dim3 grid((unsigned)((T + kPostWavesPerBlock - 1) / kPostWavesPerBlock));
  const dim3 block(kWave * kPostWavesPerBlock);
  const bool vec = (D % Store<S>::VEC == 0) && aligned16(gy) && aligned16(x) &&
                   aligned16(h_out) && aligned16(gx) && aligned16(g_hout);
  if (vec)
    hipLaunchKernelGGL((post_bwd_kernel<N, S, true>), grid, block, 0, st, (const S*)gy,
                       (const S*)x, h_res, (const S*)h_out, h_post, (S*)gx, g_hres, (S*)g_hout,
                       g_hpost, T, D);
  else
    hipLaunchKernelGGL((post_bwd_kernel<N, S, false>), grid, block, 0, st, (const S*)gy,
                       (const S*)x, h_res, (const S*)h_out, h_post, (S*)gx, g_hres, (S*)g_hout,
                       g_hpost, T, D);
  return check_launch("post_bwd");
}

template <typename S>
static int dispatch_post_fwd_n(const void* x, const float* h_res, const void* h_out,
                               const float* h_post, void* y, int64_t T, int N, int D,
                               hipStream_t st) {
  switch (N) {
    case 2: return launch_post_fwd<2, S>(x, h_res, h_out, h_post, y, T, D, st);
    case 4: return launch_post_fwd<4, S>(x, h_res, h_out, h_post, y, T, D, st);
    case 6: return launch_post_fwd<6, S>(x, h_res, h_out, h_post, y, T, D, st);
    case 8: return launch_post_fwd<8, S>(x, h_res, h_out, h_post, y, T, D, st);
  }
  return set_error(MHC_ERR_UNSUPPORTED, "mhc_post_fwd: N=%d not supported (2, 4, 6, 8)", N);
}

template <typename S>
static int dispatch_post_bwd_n(const void* gy, const void* x, const float* h_res,
                               const void* h_out, const float* h_post, void* gx, float* g_hres,
                               void* g_hout, float* g_hpost, int64_t T, int N, int D,
                               hipStream_t st) {
  switch (N) {
    case 2: return launch_post_bwd<2, S>(gy, x, h_res, h_out, h_post, gx, g_hres, g_hout, g_hpost, T, D, st);
    case 4: return launch_post_bwd<4, S>(gy, x, h_res, h_out, h_post, gx, g_hres, g_hout, g_hpost, T, D, st);
    case 6: return launch_post_bwd<6, S>(gy, x, h_res, h_out, h_post, gx, g_hres, g_hout, g_hpost, T, D, st);
    case 8: return launch_post_bwd<8, S>(gy, x, h_res, h_out, h_post, gx, g_hres, g_hout, g_hpost, T, D, st);
  }
  return set_error(MHC_ERR_UNSUPPORTED, "mhc_post_bwd: N=%d not supported (2, 4, 6, 8)", N);
}

}  // namespace mhc

using namespace mhc;

extern "C" int mhc_post_fwd(const void* x, const float* h_res, const void* h_out,
                            const float* h_post, void* y, int64_t T, int32_t N, int32_t D,
                            int32_t dtype, void* stream) {
  clear_error();
  if (T < 0 || D <= 0) return set_error(MHC_ERR_INVALID, "mhc_post_fwd: bad shape T=%lld D=%d", (long long)T, D);
  if (T == 0) return MHC_OK;
  if (!x || !h_res || !h_out || !h_post || !y) return set_error(MHC_ERR_INVALID, "mhc_post_fwd: null pointer");
  hipStream_t st = (hipStream_t)stream;
  switch (dtype) {
    case MHC_DTYPE_BF16: return dispatch_post_fwd_n<bf16_t>(x, h_res, h_out, h_post, y, T, N, D, st);
    case MHC_DTYPE_F16: return dispatch_post_fwd_n<f16_t>(x, h_res, h_out, h_post, y, T, N, D, st);
    case MHC_DTYPE_F32: return dispatch_post_fwd_n<float>(x, h_res, h_out, h_post, y, T, N, D, st);
  }
  return set_error(MHC_ERR_UNSUPPORTED, "mhc_post_fwd: dtype %d not supported", dtype);
}

extern "C" int mhc_post_bwd(const void* grad_y, const void* x, const float* h_res,
                            const void* h_out, const float* h_post, void* grad_x,
                            float* grad_h_res, void* grad_h_out, float* grad_h_post, int64_t T,
                            int32_t N, int32_t D, int32_t dtype, void* stream) {
  clear_error();
  if (T < 0 || D <= 0) return set_error(MHC_ERR_INVALID, "mhc_post_bwd: bad shape T=%lld D=%d", (long long)T, D);
  if (T == 0) return MHC_OK;
  if (!grad_y || !x || !h_res || !h_out || !h_post || !grad_x || !grad_h_res || !grad_h_out || !grad_h_post)
    return set_error(MHC_ERR_INVALID, "mhc_post_bwd: null pointer");
  hipStream_t st = (hipStream_t)stream;
  switch (dtype) {
    case MHC_DTYPE_BF16: return dispatch_post_bwd_n<bf16_t>(grad_y, x, h_res, h_out, h_post, grad_x, grad_h_res, grad_h_out, grad_h_post, T, N, D, st);
    case MHC_DTYPE_F16: return dispatch_post_bwd_n<f16_t>(grad_y, x, h_res, h_out, h_post, grad_x, grad_h_res, grad_h_out, grad_h_post, T, N, D, st);
    case MHC_DTYPE_F32: return dispatch_post_bwd_n<float>(grad_y, x, h_res, h_out, h_post, grad_x, grad_h_res, grad_h_out, grad_h_post, T, N, D, st);
  }
  return set_error(MHC_ERR_UNSUPPORTED, "mhc_post_bwd: dtype %d not supported", dtype);
}
