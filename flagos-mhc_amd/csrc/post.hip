// mhc_post forward and backward: streaming kernels over tokens.
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
// (T, D); gates are fp32 (T, N, N) and (T, N).  Three forms, chosen by shape
// (see kPostStreamMinT / kPostBlockMinD): a block of waves per token (the
// waves split D), a wave per token (backward, N > 4), and for N = 4 bf16 an
// LDS-pipelined wave per token.  In each, the N*N + N gates are uniform
// scalar loads, every lane streams 16-byte vectors of each of the N rows
// (non-temporal loads: each input is read once), accumulates in fp32 and
// stores with round-to-nearest-even (streaming stores: outputs are not
// re-read here).  The backward's N*N + N dot products
// are reduced across the wave (and the block) once per token and written by
// plain stores (no atomics), so results are deterministic.
#include <type_traits>

#include "common.hpp"
#include "lds_dma.hpp"
#include "mhc_launch.hpp"

namespace mhc {

constexpr int kPostWavesPerBlock = 4;

// MINW: waves per SIMD the register allocation must allow (2 caps the
// kernel at 256 VGPRs).
// SUM: the incoming gradient is gy + gy2 (two tensors of gy's layout, added
// in fp32 as they are read).
template <int N, typename S, bool VECTOR, int MINW = 1, bool SUM = false>
__global__ __launch_bounds__(256, MINW) void post_bwd_kernel(
    const S* __restrict__ gy, const S* __restrict__ x, const float* __restrict__ h_res,
    const S* __restrict__ h_out, const float* __restrict__ h_post, S* __restrict__ gx,
    float* __restrict__ g_hres, S* __restrict__ g_hout, float* __restrict__ g_hpost,
    int64_t T, int D, const S* __restrict__ gy2) {
  const int lane = threadIdx.x & (kWave - 1);
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int64_t t = xcd_contig(blockIdx.x, gridDim.x) * kPostWavesPerBlock + wave;
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

  if constexpr (VECTOR && N == 8 && std::is_same<S, bf16_t>::value && !SUM) {
    // N = 8: the N*N + N dot products take v_dot2_f32_bf16 on the packed
    // rows (two bf16 products and an fp32 add per instruction, no unpacking
    // of x and h_out); only grad_y is unpacked, for grad_x and grad_h_out
    constexpr int V = 8;
    auto dot2 = [](uint32_t a, uint32_t b, float c) {
      return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, a), __builtin_bit_cast(bf16x2_t, b), c,
                                             false);
    };
    for (int d = lane * V; d < D; d += kWave * V) {
      u32x4 graw[N], xraw[N];
#pragma unroll
      for (int i = 0; i < N; ++i) graw[i] = ld16nt(gy + xrow + (int64_t)i * D + d);
#pragma unroll
      for (int j = 0; j < N; ++j) xraw[j] = ld16nt(x + xrow + (int64_t)j * D + d);
      const u32x4 hraw = ld16nt(h_out + hrow + d);
      float gv[N][V];
#pragma unroll
      for (int i = 0; i < N; ++i) Store<S>::unpack(graw[i], gv[i]);
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
      for (int w = 0; w < 4; ++w) {
#pragma unroll
        for (int j = 0; j < N; ++j)
#pragma unroll
          for (int i = 0; i < N; ++i) acc_r[j * N + i] = dot2(xraw[j][w], graw[i][w], acc_r[j * N + i]);
#pragma unroll
        for (int i = 0; i < N; ++i) acc_p[i] = dot2(hraw[w], graw[i][w], acc_p[i]);
      }
    }
  } else if constexpr (VECTOR) {
    constexpr int V = Store<S>::VEC;
    for (int d = lane * V; d < D; d += kWave * V) {
      float gv[N][V], xv[N][V], hv[V];
#pragma unroll
      for (int i = 0; i < N; ++i) Store<S>::unpack(ld16nt(gy + xrow + (int64_t)i * D + d), gv[i]);
      if constexpr (SUM) {
#pragma unroll
        for (int i = 0; i < N; ++i) {
          float g2[V];
          Store<S>::unpack(ld16nt(gy2 + xrow + (int64_t)i * D + d), g2);
#pragma unroll
          for (int e = 0; e < V; ++e) gv[i][e] += g2[e];
        }
      }
#pragma unroll
      for (int j = 0; j < N; ++j) Store<S>::unpack(ld16nt(x + xrow + (int64_t)j * D + d), xv[j]);
      Store<S>::unpack(ld16nt(h_out + hrow + d), hv);
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
      for (int i = 0; i < N; ++i) {
        gv[i] = load_elem(gy, xrow + (int64_t)i * D + d);
        if constexpr (SUM) gv[i] += load_elem(gy2, xrow + (int64_t)i * D + d);
      }
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

  {
    // the wave's totals: value k + rho * RP / 4 in row rho of acc[k]
    constexpr int R = N * N + N, RP = (R + 3) / 4 * 4;
    float acc[RP];
#pragma unroll
    for (int i = 0; i < RP; ++i) acc[i] = i < N * N ? acc_r[i < N * N ? i : 0] : i < R ? acc_p[i < R ? i - N * N : 0] : 0.f;
    wave_sum_rows<RP>(acc);
    if ((lane & 15) == 0) {
      const int base = (lane >> 4) * (RP / 4);
#pragma unroll
      for (int k = 0; k < RP / 4; ++k) {
        const int i = base + k;
        if (i < N * N)
          g_hres[t * (N * N) + i] = acc[k];
        else if (i < R)
          g_hpost[t * N + i - N * N] = acc[k];
      }
    }
  }
}

// ---------------------------------------------------------------------------
// Block forms: a block of W = min(16 forward / 8 backward, chunks) waves per
// token, the waves splitting D into 64 * V-column chunks (wave w takes chunks
// w, w + W, ...), so all of a token's loads are in flight at once.  With a
// wave per token a call with few tokens runs a handful of waves, each
// streaming its whole token serially (T = 1, N = 4, D = 7168: 11 us forward,
// 19 us backward, against 3.3 and 6.4 us here).  At large T the block forms
// also beat the LDS-pipelined kernels below for D >= 2048 (D = 7168 on one
// MI355X: backward 2.23 against 2.50 ms, forward 1.48 against 1.60 ms): only
// a few tokens per CU are in flight, each read as a few long contiguous
// streams.  Inputs are read once, so loads are non-temporal (measured 3-7%
// faster than default loads here).  Every output element of the forward, grad_x and grad_h_out uses
// the FMA order of the other kernels (bit-identical results); the backward's
// N * N + N dot products are summed per lane over its chunks, across the wave
// (wave_sum_rows), then over the waves in order through LDS (no atomics).
// ---------------------------------------------------------------------------
constexpr int kPostBlockWaves = 8;     // backward: 132 VGPRs at N = 4 allow 8 waves
constexpr int kPostFwdBlockWaves = 16;  // forward: 68 VGPRs

template <int N, typename S, bool VECTOR>
__global__ __launch_bounds__(kWave * kPostFwdBlockWaves) void post_fwd_block_kernel(
    const S* __restrict__ x, const float* __restrict__ h_res, const S* __restrict__ h_out,
    const float* __restrict__ h_post, S* __restrict__ y, int D) {
  constexpr int V = VECTOR ? Store<S>::VEC : 1, CW = kWave * V;
  const int lane = threadIdx.x & (kWave - 1);
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int W = blockDim.x / kWave;
  // XCD-contiguous order at N = 4 (c5: 1447 -> 1360 us); N = 8 rows (D =
  // 2048, config 4) measured faster in the plain order (380 against 397 us)
  const int64_t t = N == 4 ? xcd_contig(blockIdx.x, gridDim.x) : (int64_t)blockIdx.x;
  float hr[N * N], hp[N];
#pragma unroll
  for (int i = 0; i < N * N; ++i) hr[i] = h_res[t * (N * N) + i];
#pragma unroll
  for (int i = 0; i < N; ++i) hp[i] = h_post[t * N + i];
  const int64_t xrow = t * (int64_t)N * D, hrow = t * (int64_t)D;
  for (int d = wave * CW + lane * V; d < D; d += W * CW) {
    float xv[N][V], hv[V];
    if constexpr (VECTOR) {
#pragma unroll
      for (int j = 0; j < N; ++j) Store<S>::unpack(ld16nt(x + xrow + (int64_t)j * D + d), xv[j]);
      Store<S>::unpack(ld16nt(h_out + hrow + d), hv);
    } else {
#pragma unroll
      for (int j = 0; j < N; ++j) xv[j][0] = load_elem(x, xrow + (int64_t)j * D + d);
      hv[0] = load_elem(h_out, hrow + d);
    }
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
      if constexpr (VECTOR)
        st16nt(y + xrow + (int64_t)i * D + d, Store<S>::pack(o));
      else
        store_elem(y, xrow + (int64_t)i * D + d, o[0]);
    }
  }
}

// MINW: waves per SIMD the registers must allow (4 = two 8-wave blocks per CU)
template <int N, typename S, bool VECTOR, bool SUM = false, int MINW = 1>  // SUM as in post_bwd_kernel
__global__ __launch_bounds__(kWave * kPostBlockWaves, MINW) void post_bwd_block_kernel(
    const S* __restrict__ gy, const S* __restrict__ x, const float* __restrict__ h_res,
    const S* __restrict__ h_out, const float* __restrict__ h_post, S* __restrict__ gx,
    float* __restrict__ g_hres, S* __restrict__ g_hout, float* __restrict__ g_hpost, int D,
    const S* __restrict__ gy2) {
  constexpr int V = VECTOR ? Store<S>::VEC : 1, CW = kWave * V, R = N * N + N;
  __shared__ float red[kPostBlockWaves][R];
  const int lane = threadIdx.x & (kWave - 1);
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int W = blockDim.x / kWave;
  const int64_t t = blockIdx.x;  // (XCD-contiguous order measured 2.5% slower here at c5)
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
  const int64_t xrow = t * (int64_t)N * D, hrow = t * (int64_t)D;
  for (int d = wave * CW + lane * V; d < D; d += W * CW) {
    float gv[N][V], xv[N][V], hv[V];
    if constexpr (VECTOR) {
#pragma unroll
      for (int i = 0; i < N; ++i) Store<S>::unpack(ld16nt(gy + xrow + (int64_t)i * D + d), gv[i]);
      if constexpr (SUM) {
#pragma unroll
        for (int i = 0; i < N; ++i) {
          float g2[V];
          Store<S>::unpack(ld16nt(gy2 + xrow + (int64_t)i * D + d), g2);
#pragma unroll
          for (int e = 0; e < V; ++e) gv[i][e] += g2[e];
        }
      }
#pragma unroll
      for (int j = 0; j < N; ++j) Store<S>::unpack(ld16nt(x + xrow + (int64_t)j * D + d), xv[j]);
      Store<S>::unpack(ld16nt(h_out + hrow + d), hv);
    } else {
#pragma unroll
      for (int i = 0; i < N; ++i) {
        gv[i][0] = load_elem(gy, xrow + (int64_t)i * D + d);
        if constexpr (SUM) gv[i][0] += load_elem(gy2, xrow + (int64_t)i * D + d);
      }
#pragma unroll
      for (int j = 0; j < N; ++j) xv[j][0] = load_elem(x, xrow + (int64_t)j * D + d);
      hv[0] = load_elem(h_out, hrow + d);
    }
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
      if constexpr (VECTOR)
        st16nt(gx + xrow + (int64_t)j * D + d, Store<S>::pack(o));
      else
        store_elem(gx, xrow + (int64_t)j * D + d, o[0]);
    }
    float oh[V];
#pragma unroll
    for (int e = 0; e < V; ++e) {
      float a = 0.f;
#pragma unroll
      for (int i = 0; i < N; ++i) a = fmaf(hp[i], gv[i][e], a);
      oh[e] = a;
    }
    if constexpr (VECTOR)
      st16nt(g_hout + hrow + d, Store<S>::pack(oh));
    else
      store_elem(g_hout, hrow + d, oh[0]);
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
  {
    // the wave's totals: value k + rho * RP / 4 in row rho of acc[k]
    constexpr int RP = (R + 3) / 4 * 4;
    float acc[RP];
#pragma unroll
    for (int i = 0; i < RP; ++i) acc[i] = i < N * N ? acc_r[i < N * N ? i : 0] : i < R ? acc_p[i < R ? i - N * N : 0] : 0.f;
    wave_sum_rows<RP>(acc);
    if ((lane & 15) == 0) {
      const int base = (lane >> 4) * (RP / 4);
#pragma unroll
      for (int k = 0; k < RP / 4; ++k)
        if (base + k < R) red[wave][base + k] = acc[k];
    }
  }
  __syncthreads();
  for (int r = threadIdx.x; r < R; r += blockDim.x) {  // R = 72 > 64 threads at N = 8, W = 1
    float v = red[0][r];
    for (int w = 1; w < W; ++w) v += red[w][r];
    if (r < N * N)
      g_hres[t * (N * N) + r] = v;
    else
      g_hpost[t * N + r - N * N] = v;
  }
}

// Waves per block: one per 64 * V-column chunk, at most `cap`.
static inline int post_block_waves(int D, int V, int cap) {
  const int chunks = (D + kWave * V - 1) / (kWave * V);
  return chunks < cap ? chunks : cap;
}

// Kernel choice (measured on MI355X): the LDS-pipelined kernels (N = 4 bf16)
// and the wave-per-token backward (other shapes) need at least
// kPostStreamMinT tokens to fill the chip; for N = 4 bf16 the LDS-pipelined
// kernels win only for D < kPostBlockMinD.  The wave-per-token backward stays
// for N > 4 at large T (the block form needs 225 VGPRs at N = 8 and ran 1.5x
// slower at D = 2048).
// (A/B on one box, N = 4 bf16, forward / backward us, LDS-pipelined -> block:
// bench.py at D = 2048 T = 32768 216 -> 202 / 331-336 -> 293, D = 4096
// T = 16384 208 -> 206 / 325 -> 319; a timing loop at D = 1024 T = 16384
// 50 -> 55 / 80 -> 80, D = 3072 161 -> 154 / 249 -> 236.)
constexpr int64_t kPostStreamMinT = 1024;
constexpr int kPostBlockMinD = 2048;

// ---------------------------------------------------------------------------
// LDS-pipelined forms (bf16, 16-byte aligned rows, D % 8 == 0)
//
// Same arithmetic, but the input rows reach the lanes through direct-to-LDS
// loads: every wave of a persistent grid owns a ring of S slots in
// LDS, one slot = the R input rows of one token over 512 columns (one 1 KB
// load per row, lane l -> columns 8l..8l+7), issued S-1 slots
// ahead, so the loads in flight hold no registers and a wave keeps ~3 slots
// of reads outstanding while it computes and stores.  A wave reads back only
// what its own loads wrote (no barriers).  Columns >= D load as zero through
// the buffer range check and their stores are dropped.  Wave w of the grid
// takes the tokens w, w + W, ... (W waves in all), all column blocks of a
// token in a row.  Gates are wave-uniform scalar loads (lgkmcnt, outside the
// vector-memory pipeline).  Measured on the MI355X, this path moves mixed
// read/write traffic ~7% faster than register loads.
// ---------------------------------------------------------------------------
constexpr int kPostFwdStages = 4;  // 4 waves x 4 slots x 5 KB: two blocks per CU
constexpr int kPostBwdStages = 4;  // 4 waves x 4 slots x 9 KB: one block per CU

template <int N>
__global__ __launch_bounds__(256) void post_fwd_dma_kernel(const bf16_t* __restrict__ x,
                                                           const float* __restrict__ h_res,
                                                           const bf16_t* __restrict__ h_out,
                                                           const float* __restrict__ h_post,
                                                           bf16_t* __restrict__ y, int64_t T, int D) {
  constexpr int R = N + 1, S = kPostFwdStages;  // slot rows: x[0..N-1], h_out
  constexpr int VM_START = (S - 2) * R, VM_STEADY = (S - 2) * R + (S - 1) * N;
  static_assert(VM_STEADY < 64, "vmcnt range");
  __shared__ u32x4 ring[kPostWavesPerBlock * S * R * kWave];
  const int lane = threadIdx.x & (kWave - 1);
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int64_t gw = (int64_t)blockIdx.x * kPostWavesPerBlock + wave, W = (int64_t)gridDim.x * kPostWavesPerBlock;
  const int ncb = (D + 511) / 512;
  const int64_t ntok = (T - gw + W - 1) / W;
  if (ntok <= 0) return;  // this wave only: no barriers below
  const int64_t J = ntok * ncb;
  const uint32_t wring = lds_addr(ring) + (uint32_t)(wave * S * R * 1024);
  const int64_t ND = (int64_t)N * D;

  int64_t itok = gw;
  int icb = 0;
  auto issue = [&](int64_t j) {
    const uint32_t slot = wring + (uint32_t)((j % S) * R * 1024);
    const int col = icb * 512 + 8 * lane;
    const auto rx = rows_rsrc(x + itok * ND, ND * 2);
    const auto rh = rows_rsrc(h_out + itok * D, (int64_t)D * 2);
#pragma unroll
    for (int n = 0; n < N; ++n)
      __builtin_amdgcn_raw_ptr_buffer_load_lds(rx, (lds_void_t*)(uintptr_t)(slot + n * 1024), 16,
                                               col < D ? (uint32_t)(((int64_t)n * D + col) * 2) : kBufferOob,
                                               0, 0, 2 /* nt */);
    __builtin_amdgcn_raw_ptr_buffer_load_lds(rh, (lds_void_t*)(uintptr_t)(slot + N * 1024), 16,
                                             col < D ? (uint32_t)(col * 2) : kBufferOob, 0, 0, 2);
    if (++icb == ncb) {
      icb = 0;
      itok += W;
    }
  };
  for (int64_t j = 0; j < S - 1 && j < J; ++j) issue(j);

  int64_t ctok = gw;
  int ccb = 0;
  float hr[N * N], hp[N];
  auto gates = [&]() {
#pragma unroll
    for (int i = 0; i < N * N; ++i) hr[i] = h_res[ctok * (N * N) + i];
#pragma unroll
    for (int i = 0; i < N; ++i) hp[i] = h_post[ctok * N + i];
  };
  gates();
  for (int64_t j = 0; j < J; ++j) {
    // this wave's loads of slot j have landed once at most V newer vector
    // memory operations are outstanding
    if (j + S - 2 < J) {
      if (j >= S - 1)
        wait_vmcnt<VM_STEADY>();
      else
        wait_vmcnt<VM_START>();
    } else {
      wait_vmcnt<0>();
    }
    asm volatile("" ::: "memory");
    // the next loads reuse the slot this wave read (and waited for) last iteration
    if (j + S - 1 < J) issue(j + S - 1);
    u32x4 v[R];
    read_slot<R>(v, wring + (uint32_t)((j % S) * R * 1024) + lane * 16);
    float xv[N][8], hv[8];
#pragma unroll
    for (int n = 0; n < N; ++n) Store<bf16_t>::unpack(v[n], xv[n]);
    Store<bf16_t>::unpack(v[N], hv);
    const int col = ccb * 512 + 8 * lane;
    const auto ry = rows_rsrc(y + ctok * ND, ND * 2);
#pragma unroll
    for (int i = 0; i < N; ++i) {
      float o[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        float acc = hp[i] * hv[e];
#pragma unroll
        for (int jj = 0; jj < N; ++jj) acc = fmaf(hr[jj * N + i], xv[jj][e], acc);
        o[e] = acc;
      }
      __builtin_amdgcn_raw_buffer_store_b128(Store<bf16_t>::pack(o), ry,
                                             col < D ? (uint32_t)(((int64_t)i * D + col) * 2) : kBufferOob, 0,
                                             2 /* nt */);
    }
    if (++ccb == ncb) {
      ccb = 0;
      ctok += W;
      if (ctok < T) gates();
    }
  }
}

template <int N>
__global__ __launch_bounds__(256) void post_bwd_dma_kernel(
    const bf16_t* __restrict__ gy, const bf16_t* __restrict__ x, const float* __restrict__ h_res,
    const bf16_t* __restrict__ h_out, const float* __restrict__ h_post, bf16_t* __restrict__ gx,
    float* __restrict__ g_hres, bf16_t* __restrict__ g_hout, float* __restrict__ g_hpost, int64_t T,
    int D) {
  constexpr int R = 2 * N + 1, S = kPostBwdStages;  // slot rows: gy[0..N-1], x[0..N-1], h_out
  constexpr int VM_START = (S - 2) * R, VM_STEADY = (S - 2) * R + (S - 1) * (N + 1);
  static_assert(VM_STEADY < 64, "vmcnt range");
  __shared__ u32x4 ring[kPostWavesPerBlock * S * R * kWave];
  const int lane = threadIdx.x & (kWave - 1);
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int64_t gw = (int64_t)blockIdx.x * kPostWavesPerBlock + wave, W = (int64_t)gridDim.x * kPostWavesPerBlock;
  const int ncb = (D + 511) / 512;
  const int64_t ntok = (T - gw + W - 1) / W;
  if (ntok <= 0) return;  // this wave only: no barriers below
  const int64_t J = ntok * ncb;
  const uint32_t wring = lds_addr(ring) + (uint32_t)(wave * S * R * 1024);
  const int64_t ND = (int64_t)N * D;

  int64_t itok = gw;
  int icb = 0;
  auto issue = [&](int64_t j) {
    const uint32_t slot = wring + (uint32_t)((j % S) * R * 1024);
    const int col = icb * 512 + 8 * lane;
    const auto rg = rows_rsrc(gy + itok * ND, ND * 2);
    const auto rx = rows_rsrc(x + itok * ND, ND * 2);
    const auto rh = rows_rsrc(h_out + itok * D, (int64_t)D * 2);
#pragma unroll
    for (int n = 0; n < N; ++n) {
      const uint32_t off = col < D ? (uint32_t)(((int64_t)n * D + col) * 2) : kBufferOob;
      __builtin_amdgcn_raw_ptr_buffer_load_lds(rg, (lds_void_t*)(uintptr_t)(slot + n * 1024), 16, off, 0, 0, 2);
      __builtin_amdgcn_raw_ptr_buffer_load_lds(rx, (lds_void_t*)(uintptr_t)(slot + (N + n) * 1024), 16, off, 0, 0,
                                               2);
    }
    __builtin_amdgcn_raw_ptr_buffer_load_lds(rh, (lds_void_t*)(uintptr_t)(slot + 2 * N * 1024), 16,
                                             col < D ? (uint32_t)(col * 2) : kBufferOob, 0, 0, 2);
    if (++icb == ncb) {
      icb = 0;
      itok += W;
    }
  };
  for (int64_t j = 0; j < S - 1 && j < J; ++j) issue(j);

  int64_t ctok = gw;
  int ccb = 0;
  float hr[N * N], hp[N], acc_r[N * N], acc_p[N];
  auto gates = [&]() {
#pragma unroll
    for (int i = 0; i < N * N; ++i) hr[i] = h_res[ctok * (N * N) + i];
#pragma unroll
    for (int i = 0; i < N; ++i) hp[i] = h_post[ctok * N + i];
#pragma unroll
    for (int i = 0; i < N * N; ++i) acc_r[i] = 0.f;
#pragma unroll
    for (int i = 0; i < N; ++i) acc_p[i] = 0.f;
  };
  gates();
  for (int64_t j = 0; j < J; ++j) {
    if (j + S - 2 < J) {
      if (j >= S - 1)
        wait_vmcnt<VM_STEADY>();
      else
        wait_vmcnt<VM_START>();
    } else {
      wait_vmcnt<0>();
    }
    asm volatile("" ::: "memory");
    if (j + S - 1 < J) issue(j + S - 1);
    u32x4 v[R];
    read_slot<R>(v, wring + (uint32_t)((j % S) * R * 1024) + lane * 16);
    float gv[N][8], xv[N][8], hv[8];
#pragma unroll
    for (int n = 0; n < N; ++n) {
      Store<bf16_t>::unpack(v[n], gv[n]);
      Store<bf16_t>::unpack(v[N + n], xv[n]);
    }
    Store<bf16_t>::unpack(v[2 * N], hv);
    const int col = ccb * 512 + 8 * lane;
    const auto rgx = rows_rsrc(gx + ctok * ND, ND * 2);
#pragma unroll
    for (int jj = 0; jj < N; ++jj) {
      float o[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        float a = 0.f;
#pragma unroll
        for (int i = 0; i < N; ++i) a = fmaf(hr[jj * N + i], gv[i][e], a);
        o[e] = a;
      }
      __builtin_amdgcn_raw_buffer_store_b128(Store<bf16_t>::pack(o), rgx,
                                             col < D ? (uint32_t)(((int64_t)jj * D + col) * 2) : kBufferOob, 0,
                                             2);
    }
    {
      float oh[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        float a = 0.f;
#pragma unroll
        for (int i = 0; i < N; ++i) a = fmaf(hp[i], gv[i][e], a);
        oh[e] = a;
      }
      const auto rgh = rows_rsrc(g_hout + ctok * D, (int64_t)D * 2);
      __builtin_amdgcn_raw_buffer_store_b128(Store<bf16_t>::pack(oh), rgh, col < D ? (uint32_t)(col * 2) : kBufferOob,
                                             0, 2);
    }
#pragma unroll
    for (int e = 0; e < 8; ++e) {
#pragma unroll
      for (int jj = 0; jj < N; ++jj)
#pragma unroll
        for (int i = 0; i < N; ++i) acc_r[jj * N + i] = fmaf(xv[jj][e], gv[i][e], acc_r[jj * N + i]);
#pragma unroll
      for (int i = 0; i < N; ++i) acc_p[i] = fmaf(hv[e], gv[i][e], acc_p[i]);
    }
    if (++ccb == ncb) {
      // token done: reduce the N*N + N dot products across the wave (value
      // k + rho * RP / 4 in row rho of acc[k]); these stores only add vector
      // memory operations newer than the counted ones
      constexpr int R2 = N * N + N, RP = (R2 + 3) / 4 * 4;
      float acc[RP];
#pragma unroll
      for (int i = 0; i < RP; ++i)
        acc[i] = i < N * N ? acc_r[i < N * N ? i : 0] : i < R2 ? acc_p[i < R2 ? i - N * N : 0] : 0.f;
      wave_sum_rows<RP>(acc);
      if ((lane & 15) == 0) {
        const int base = (lane >> 4) * (RP / 4);
#pragma unroll
        for (int k = 0; k < RP / 4; ++k) {
          const int i = base + k;
          if (i < N * N)
            g_hres[ctok * (N * N) + i] = acc[k];
          else if (i < R2)
            g_hpost[ctok * N + i - N * N] = acc[k];
        }
      }
      ccb = 0;
      ctok += W;
      if (ctok < T) gates();
    }
  }
}

// Persistent grid: as many blocks as fit on the device at once (the LDS rings
// bound the residency), at most one wave per token.
template <typename K>
static int64_t post_dma_grid(K kernel, int64_t T) {
  int per_cu = 0;
  if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, kernel, kWave * kPostWavesPerBlock, 0) != hipSuccess ||
      per_cu <= 0)
    per_cu = 1;
  const int64_t grid = (int64_t)device_cu_count() * per_cu;
  const int64_t max_grid = (T + kPostWavesPerBlock - 1) / kPostWavesPerBlock;
  return grid < max_grid ? grid : max_grid;
}

// ---------------------------------------------------------------------------
// host launchers
// ---------------------------------------------------------------------------
template <int N, typename S>
static int launch_post_fwd(const void* x, const float* h_res, const void* h_out,
                           const float* h_post, void* y, int64_t T, int D, hipStream_t st) {
  const dim3 block(kWave * kPostWavesPerBlock);
  const bool vec = (D % Store<S>::VEC == 0) && aligned16(x) && aligned16(h_out) && aligned16(y);
  if constexpr (N == 4 && std::is_same<S, bf16_t>::value) {
    if (vec && T >= kPostStreamMinT && D < kPostBlockMinD) {
      const int64_t g = post_dma_grid(post_fwd_dma_kernel<N>, T);
      hipLaunchKernelGGL((post_fwd_dma_kernel<N>), dim3((unsigned)g), block, 0, st, (const bf16_t*)x, h_res,
                         (const bf16_t*)h_out, h_post, (bf16_t*)y, T, D);
      return check_launch("post_fwd_dma");
    }
  }
  const int waves = post_block_waves(D, vec ? Store<S>::VEC : 1, kPostFwdBlockWaves);
  const dim3 gs((unsigned)T), bs(kWave * waves);
  // Blocks of 10 or more waves run one token per CU at a time (D = 7168 /
  // 5120: 2.6% / 1.6% faster); narrower ones (N = 8 takes this kernel at
  // every D) several to a CU (N = 8, D = 2048: 440 -> 376 us at T = 32768).
  const size_t lds = waves >= 10 ? one_block_per_cu_lds() : 0;
  if (int rc = check_grid(gs, bs, "mhc_post_fwd")) return rc;
  if (vec)
    hipLaunchKernelGGL((post_fwd_block_kernel<N, S, true>), gs, bs, lds, st, (const S*)x, h_res,
                       (const S*)h_out, h_post, (S*)y, D);
  else
    hipLaunchKernelGGL((post_fwd_block_kernel<N, S, false>), gs, bs, lds, st, (const S*)x, h_res,
                       (const S*)h_out, h_post, (S*)y, D);
  return check_launch("post_fwd_block");
}

// True when the LDS-pipelined kernel (which has no summed-gradient form)
// is the backward's kernel for this shape.
template <int N, typename S>
static bool post_bwd_uses_dma(int64_t T, int D, bool vec) {
  return N == 4 && std::is_same<S, bf16_t>::value && vec && T >= kPostStreamMinT && D < kPostBlockMinD;
}

// gy2 == nullptr: the gradient is gy; otherwise gy + gy2 (the block and
// wave-per-token kernels; the LDS-pipelined kernel's shapes take the block
// kernel then).
template <int N, typename S>
static int launch_post_bwd(const void* gy, const void* gy2, const void* x, const float* h_res, const void* h_out,
                           const float* h_post, void* gx, float* g_hres, void* g_hout,
                           float* g_hpost, int64_t T, int D, hipStream_t st) {
  const dim3 grid((unsigned)((T + kPostWavesPerBlock - 1) / kPostWavesPerBlock));
  const dim3 block(kWave * kPostWavesPerBlock);
  const bool vec = (D % Store<S>::VEC == 0) && aligned16(gy) && aligned16(x) &&
                   aligned16(h_out) && aligned16(gx) && aligned16(g_hout) && (!gy2 || aligned16(gy2));
  const bool sum = gy2 != nullptr;
  const bool dma = post_bwd_uses_dma<N, S>(T, D, vec);
  const bool block_form = T < kPostStreamMinT || (N <= 4 && !dma) || (sum && dma);
  const S* g2 = static_cast<const S*>(gy2);
  if (block_form) {
    const dim3 gs((unsigned)T), bs(kWave * post_block_waves(D, vec ? Store<S>::VEC : 1, kPostBlockWaves));
    if (int rc = check_grid(gs, bs, "mhc_post_bwd")) return rc;
    if (sum) {
      if (vec)
        hipLaunchKernelGGL((post_bwd_block_kernel<N, S, true, true>), gs, bs, 0, st, (const S*)gy, (const S*)x,
                           h_res, (const S*)h_out, h_post, (S*)gx, g_hres, (S*)g_hout, g_hpost, D, g2);
      else
        hipLaunchKernelGGL((post_bwd_block_kernel<N, S, false, true>), gs, bs, 0, st, (const S*)gy, (const S*)x,
                           h_res, (const S*)h_out, h_post, (S*)gx, g_hres, (S*)g_hout, g_hpost, D, g2);
    } else {
      if (vec) {
        // N = 4 with exactly one 512-column chunk per wave (D in (3584, 4096]):
        // capped at 128 registers (a 20-byte spill) two blocks share a CU and
        // one token's reduction overlaps the next one's loads (bench.py at D =
        // 4096, T = 16384: 337-342 -> 319-322 us); with two chunks a wave (D =
        // 7168: 2.19-2.22 -> 2.32-2.33 ms) or four waves (D = 2048: 293 -> 311
        // us) the cap is slower
        if (N == 4 && (D + 511) / 512 == kPostBlockWaves)
          hipLaunchKernelGGL((post_bwd_block_kernel<N, S, true, false, 4>), gs, bs, 0, st, (const S*)gy,
                             (const S*)x, h_res, (const S*)h_out, h_post, (S*)gx, g_hres, (S*)g_hout, g_hpost,
                             D, g2);
        else
          hipLaunchKernelGGL((post_bwd_block_kernel<N, S, true>), gs, bs, 0, st, (const S*)gy, (const S*)x,
                             h_res, (const S*)h_out, h_post, (S*)gx, g_hres, (S*)g_hout, g_hpost, D, g2);
      } else {
        hipLaunchKernelGGL((post_bwd_block_kernel<N, S, false>), gs, bs, 0, st, (const S*)gy, (const S*)x,
                           h_res, (const S*)h_out, h_post, (S*)gx, g_hres, (S*)g_hout, g_hpost, D, g2);
      }
    }
    return check_launch("post_bwd_block");
  }
  if constexpr (N == 4 && std::is_same<S, bf16_t>::value) {
    if (dma) {
      const int64_t g = post_dma_grid(post_bwd_dma_kernel<N>, T);
      hipLaunchKernelGGL((post_bwd_dma_kernel<N>), dim3((unsigned)g), block, 0, st, (const bf16_t*)gy,
                         (const bf16_t*)x, h_res, (const bf16_t*)h_out, h_post, (bf16_t*)gx, g_hres,
                         (bf16_t*)g_hout, g_hpost, T, D);
      return check_launch("post_bwd_dma");
    }
  }
  if (sum) {
    if (vec)
      hipLaunchKernelGGL((post_bwd_kernel<N, S, true, 1, true>), grid, block, 0, st, (const S*)gy,
                         (const S*)x, h_res, (const S*)h_out, h_post, (S*)gx, g_hres, (S*)g_hout,
                         g_hpost, T, D, g2);
    else
      hipLaunchKernelGGL((post_bwd_kernel<N, S, false, 1, true>), grid, block, 0, st, (const S*)gy,
                         (const S*)x, h_res, (const S*)h_out, h_post, (S*)gx, g_hres, (S*)g_hout,
                         g_hpost, T, D, g2);
    return check_launch("post_bwd");
  }
  if constexpr (N == 8) {
    // 270 VGPRs leave one wave per SIMD; capped at 256 (a 60-byte spill) two
    // fit, which pays at narrow rows (D = 2048, T = 32768: 729 -> 629 us) but
    // not wider ones (D = 4096: 706 -> 756 us; D = 7168: equal)
    if (vec && D <= 2048) {
      hipLaunchKernelGGL((post_bwd_kernel<N, S, true, 2>), grid, block, 0, st, (const S*)gy, (const S*)x, h_res,
                         (const S*)h_out, h_post, (S*)gx, g_hres, (S*)g_hout, g_hpost, T, D, g2);
      return check_launch("post_bwd");
    }
  }
  if (vec)
    hipLaunchKernelGGL((post_bwd_kernel<N, S, true>), grid, block, 0, st, (const S*)gy,
                       (const S*)x, h_res, (const S*)h_out, h_post, (S*)gx, g_hres, (S*)g_hout,
                       g_hpost, T, D, g2);
  else
    hipLaunchKernelGGL((post_bwd_kernel<N, S, false>), grid, block, 0, st, (const S*)gy,
                       (const S*)x, h_res, (const S*)h_out, h_post, (S*)gx, g_hres, (S*)g_hout,
                       g_hpost, T, D, g2);
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
static int dispatch_post_bwd_n(const void* gy, const void* gy2, const void* x, const float* h_res,
                               const void* h_out, const float* h_post, void* gx, float* g_hres,
                               void* g_hout, float* g_hpost, int64_t T, int N, int D,
                               hipStream_t st) {
  switch (N) {
    case 2: return launch_post_bwd<2, S>(gy, gy2, x, h_res, h_out, h_post, gx, g_hres, g_hout, g_hpost, T, D, st);
    case 4: return launch_post_bwd<4, S>(gy, gy2, x, h_res, h_out, h_post, gx, g_hres, g_hout, g_hpost, T, D, st);
    case 6: return launch_post_bwd<6, S>(gy, gy2, x, h_res, h_out, h_post, gx, g_hres, g_hout, g_hpost, T, D, st);
    case 8: return launch_post_bwd<8, S>(gy, gy2, x, h_res, h_out, h_post, gx, g_hres, g_hout, g_hpost, T, D, st);
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
  if (int rc = check_tokens(T, "mhc_post_fwd")) return rc;
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

static int post_bwd_entry(const char* what, const void* grad_y, const void* grad_y2, const void* x,
                          const float* h_res, const void* h_out, const float* h_post, void* grad_x,
                          float* grad_h_res, void* grad_h_out, float* grad_h_post, int64_t T, int32_t N,
                          int32_t D, int32_t dtype, void* stream) {
  clear_error();
  if (T < 0 || D <= 0) return set_error(MHC_ERR_INVALID, "%s: bad shape T=%lld D=%d", what, (long long)T, D);
  if (int rc = check_tokens(T, what)) return rc;
  if (T == 0) return MHC_OK;
  if (!grad_y || !x || !h_res || !h_out || !h_post || !grad_x || !grad_h_res || !grad_h_out || !grad_h_post)
    return set_error(MHC_ERR_INVALID, "%s: null pointer", what);
  hipStream_t st = (hipStream_t)stream;
  switch (dtype) {
    case MHC_DTYPE_BF16: return dispatch_post_bwd_n<bf16_t>(grad_y, grad_y2, x, h_res, h_out, h_post, grad_x, grad_h_res, grad_h_out, grad_h_post, T, N, D, st);
    case MHC_DTYPE_F16: return dispatch_post_bwd_n<f16_t>(grad_y, grad_y2, x, h_res, h_out, h_post, grad_x, grad_h_res, grad_h_out, grad_h_post, T, N, D, st);
    case MHC_DTYPE_F32: return dispatch_post_bwd_n<float>(grad_y, grad_y2, x, h_res, h_out, h_post, grad_x, grad_h_res, grad_h_out, grad_h_post, T, N, D, st);
  }
  return set_error(MHC_ERR_UNSUPPORTED, "%s: dtype %d not supported", what, dtype);
}

extern "C" int mhc_post_bwd(const void* grad_y, const void* x, const float* h_res,
                            const void* h_out, const float* h_post, void* grad_x,
                            float* grad_h_res, void* grad_h_out, float* grad_h_post, int64_t T,
                            int32_t N, int32_t D, int32_t dtype, void* stream) {
  return post_bwd_entry("mhc_post_bwd", grad_y, nullptr, x, h_res, h_out, h_post, grad_x, grad_h_res, grad_h_out,
                        grad_h_post, T, N, D, dtype, stream);
}

extern "C" int mhc_post_bwd_sum(const void* grad_y, const void* grad_y2, const void* x, const float* h_res,
                                const void* h_out, const float* h_post, void* grad_x, float* grad_h_res,
                                void* grad_h_out, float* grad_h_post, int64_t T, int32_t N, int32_t D,
                                int32_t dtype, void* stream) {
  if (!grad_y2) {
    clear_error();
    return set_error(MHC_ERR_INVALID, "mhc_post_bwd_sum: null pointer");
  }
  return post_bwd_entry("mhc_post_bwd_sum", grad_y, grad_y2, x, h_res, h_out, h_post, grad_x, grad_h_res,
                        grad_h_out, grad_h_post, T, N, D, dtype, stream);
}

extern "C" int mhc_post_bwd_sum_fused(int64_t T, int32_t N, int32_t D, int32_t dtype) {
  // aligned rows assumed (the caller's tensors come from the allocator)
  if (N == 4 && dtype == MHC_DTYPE_BF16) return post_bwd_uses_dma<4, bf16_t>(T, D, D % 8 == 0) ? 0 : 1;
  return 1;
}
