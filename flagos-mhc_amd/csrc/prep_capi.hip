// phi preparation kernels, the library's error state and version entry points.
#include <stdarg.h>
#include <stdio.h>
#include <string.h>

#include "common.hpp"
#include "mhc_launch.hpp"
#include "pre_host.hpp"

namespace mhc {

static thread_local char g_last_error[512] = "";

int set_error(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_last_error, sizeof(g_last_error), fmt, ap);
  va_end(ap);
  return code;
}

void clear_error() { g_last_error[0] = '\0'; }

template <typename S>
__device__ __forceinline__ float phi_value(const void* phi, int64_t i) {
  return load_elem(static_cast<const S*>(phi), i);
}

// planes [P][M][ld]: plane p = bf16(phi - sum of planes < p); zero padded.
template <typename S>
__global__ void phi_planes_kernel(const void* phi, uint16_t* out, int M, int64_t K, int64_t ld,
                                  int P) {
  const int64_t total = (int64_t)M * ld;
  for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < total;
       i += (int64_t)gridDim.x * blockDim.x) {
    const int64_t m = i / ld, k = i - (i / ld) * ld;
    float v = k < K ? phi_value<S>(phi, m * K + k) : 0.f;
    for (int p = 0; p < P; ++p) {
      const uint32_t h = f32_to_bf16_bits(v);
      out[p * total + i] = (uint16_t)h;
      v -= bf16_bits_to_f32(h);
    }
  }
}

// transposed planes [P][K][MP]: out[p][k][m]
template <typename S>
__global__ void phiT_planes_kernel(const void* phi, uint16_t* out, int M, int MP, int64_t K,
                                   int P) {
  const int64_t total = K * MP;
  for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < total;
       i += (int64_t)gridDim.x * blockDim.x) {
    const int64_t k = i / MP;
    const int m = (int)(i - k * MP);
    const float v = m < M ? phi_value<S>(phi, (int64_t)m * K + k) : 0.f;
    uint32_t hi, lo;
    split2_bf16(v, hi, lo);
    out[i] = (uint16_t)hi;
    if (P > 1) out[total + i] = (uint16_t)lo;
  }
}

static unsigned grid_for(int64_t total) {
  int64_t g = (total + 255) / 256;
  if (g > 4096) g = 4096;
  if (g < 1) g = 1;
  return (unsigned)g;
}

int prepare_phi_planes(const void* phi, int32_t phi_dtype, int M, int64_t K, void* ws,
                       size_t ws_bytes, const uint16_t** planes, int64_t* ld,
                       int64_t* plane_stride, int* nplanes, hipStream_t st) {
  if (phi_dtype == MHC_DTYPE_BF16 && K % 8 == 0 && aligned16(phi)) {
    *planes = static_cast<const uint16_t*>(phi);
    *ld = K;
    *plane_stride = 0;
    *nplanes = 1;
    return MHC_OK;
  }
  const int P = phi_fwd_planes(phi_dtype);
  const int64_t L = round_up(K, 8);
  const size_t need = phi_planes_bytes(phi_dtype, M, K);
  if (!ws || ws_bytes < need)
    return set_error(MHC_ERR_INVALID, "workspace too small for phi planes (%zu < %zu bytes)",
                     ws_bytes, need);
  uint16_t* out = static_cast<uint16_t*>(ws);
  const int64_t total = (int64_t)M * L;
  switch (phi_dtype) {
    case MHC_DTYPE_BF16:
      hipLaunchKernelGGL(phi_planes_kernel<bf16_t>, dim3(grid_for(total)), dim3(256), 0, st, phi, out, M, K, L, P);
      break;
    case MHC_DTYPE_F16:
      hipLaunchKernelGGL(phi_planes_kernel<f16_t>, dim3(grid_for(total)), dim3(256), 0, st, phi, out, M, K, L, P);
      break;
    case MHC_DTYPE_F32:
      hipLaunchKernelGGL(phi_planes_kernel<float>, dim3(grid_for(total)), dim3(256), 0, st, phi, out, M, K, L, P);
      break;
    default:
      return set_error(MHC_ERR_UNSUPPORTED, "phi dtype %d not supported", phi_dtype);
  }
  *planes = out;
  *ld = L;
  *plane_stride = total;
  *nplanes = P;
  return check_launch("phi_planes");
}

int prepare_phiT_planes(const void* phi, int32_t phi_dtype, int M, int64_t K, uint16_t* dst,
                        hipStream_t st) {
  const int P = phi_bwd_planes(phi_dtype);
  const int MP = (int)round_up(M, 32);
  const int64_t total = K * MP;
  switch (phi_dtype) {
    case MHC_DTYPE_BF16:
      hipLaunchKernelGGL(phiT_planes_kernel<bf16_t>, dim3(grid_for(total)), dim3(256), 0, st, phi, dst, M, MP, K, P);
      break;
    case MHC_DTYPE_F16:
      hipLaunchKernelGGL(phiT_planes_kernel<f16_t>, dim3(grid_for(total)), dim3(256), 0, st, phi, dst, M, MP, K, P);
      break;
    case MHC_DTYPE_F32:
      hipLaunchKernelGGL(phiT_planes_kernel<float>, dim3(grid_for(total)), dim3(256), 0, st, phi, dst, M, MP, K, P);
      break;
    default:
      return set_error(MHC_ERR_UNSUPPORTED, "phi dtype %d not supported", phi_dtype);
  }
  return check_launch("phiT_planes");
}

}  // namespace mhc

extern "C" const char* mhc_last_error(void) { return mhc::g_last_error; }

extern "C" int32_t mhc_version(void) { return 100; }
