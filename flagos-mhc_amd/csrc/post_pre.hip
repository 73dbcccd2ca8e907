// Fused forward of mhc_post (layer l) and mhc_pre_clamp_sinkhorn (layer l+1).
//
// The post output x_next = h_res^T x + h_post h_out (src/mhc_post.py:344-352)
// is exactly the next layer's pre input.  Run separately, mhc_post reads x and
// writes x_next, then the pre kernel reads x_next twice (contraction, then y).
// Here the contraction stages compute x_next from x and h_out on the fly,
// write it once and feed the same bf16 values to the MFMA contraction; only
// the y pass (the pre forward's y kernel, run afterwards) reads x_next back.
// Per token that saves one full read of the N streams (N*D*2 bytes, a
// quarter of the pair's traffic).
//
// Shape: N = 4, bf16 x / h_out / phi, D a multiple of 64 and >= 256; the C
// entry point runs mhc_post then mhc_pre_clamp_sinkhorn for every other
// shape.  Where the pre forward has its single pass (T >= 8192, D = 4096 or
// 7168 .. 8192) the single-pass pre kernel runs with a post front end
// instead (post_pre_fwd_single_pass: x_next formed in the kernel, written
// once, never read back), or, if that form cannot run, post then pre.  (The tile's gates sit in one LDS buffer that wave 0 refills when it
// issues the next tile's first stage, S - 1 stages ahead: a tile must span
// at least S stages, D >= 64 * S, so that it has read its gates by then.)
//
// A block (8 waves, two per SIMD so that one wave's waits overlap the other's
// work) owns a tile of 32 tokens.  Wave w handles row block rb = w & 1
// (tokens 16rb..16rb+15) and output stream n = w >> 1.  Contraction stage s
// covers columns d in [64s, 64s+64) of all four streams, staged in LDS as
// 1 KB units filled by direct-to-LDS loads:
//   units  0..15  x[t][j][64s..64s+64]   unit 8rb + 2j + g, rows 16rb + 8g + i
//   units 16..19  h_out[t][64s..64s+64]  unit 16 + 2rb + g
//   units 20..35  phi[16mt + i][n*D + 64s + 32h + 8c]   unit 20 + 4n + 2h + mt
// An x / h_out unit holds 8 rows x 128 bytes, so each load instruction reads
// whole 128-byte row segments; slot p of a unit holds chunk
// (p & 7) ^ f(i, g) of row i = p >> 3, f(i, g) = (i >> 1) ^ 4g, which makes
// the 16 lanes of a read phase (16 rows, one chunk each) hit 16 different
// 16-byte bank groups.  A phi unit holds 16 rows (m) x 64 bytes, lane L = row
// L % 16, chunk L / 16, the MFMA B-operand layout.  Lane (r, c) of a wave
// forms x_next[t][n][64s + 32h + 8c..+8] (h = 0, 1) with the post kernel's
// fp32 FMA order and round-to-nearest-even (bit-identical to mhc_post) and
// uses the packed values as MFMA A operands (v_mfma_f32_16x16x32_bf16; B =
// phi^T of stream n).  The two halves are stored by two instructions that
// each write 8 whole 128-byte row segments: lanes r and r ^ 8 trade their
// second halves through a DPP row rotation first.  The four waves of a row
// block hold partial sums over their streams; they are added in a fixed order
// through LDS after the tile's last contraction stage, followed by heads and
// Sinkhorn exactly as in the pre kernel; pre goes to the workspace for the y
// kernel.  The y pass used to run as stages of this kernel (8 tokens x 4
// streams x 512 columns each, which needed D >= 3136 so that a y stage's
// loads followed the stores of its columns); as the block-per-token kernel
// it is faster (N = 4, D = 7168, T = 65536: 2.55 -> 2.26 ms for the fused
// forward on one MI355X).
#include "mhc_launch.hpp"
#include "pre_common.hpp"
#include "pre_host.hpp"
#include "sinkhorn.hpp"

namespace mhc {

namespace {

constexpr int kPPN = 4;
constexpr int kPPM = 2 * kPPN + kPPN * kPPN;  // 24
constexpr int kPPMT = 2;                      // 16-row m tiles (rows >= 24 load as zero)
constexpr int kPPTile = 32;                   // tokens per tile
constexpr int kPPWaves = 8;
constexpr int kPPThreads = kPPWaves * kWave;
constexpr int kPPStages = 4;                  // ring slots
constexpr int kPPCW = 64;                     // d columns per contraction stage
constexpr int kUH = 16, kUP = 20;             // first h_out / phi unit of a contraction slot
constexpr int kPPUnits = 36;                  // 1 KB units per slot
constexpr int kPPCImax = (kPPUnits + kPPWaves - 1) / kPPWaves;  // 5: loads of waves 0..3
constexpr int kPPCImin = kPPUnits / kPPWaves;                   // 4: loads of waves 4..7
constexpr int kPPCST = 2;                     // x_next stores per lane and contraction stage
constexpr int kPPMinD = kPPCW * kPPStages;    // 256: a tile spans at least S stages (gates buffer)

struct PostPreArgs {
  const bf16_t* x;       // (T, 4, D)
  const float* h_res;    // (T, 4, 4)
  const bf16_t* h_out;   // (T, D)
  const float* h_post;   // (T, 4)
  const uint16_t* phi;   // (M, 4D) bf16
  const float* alpha;
  const float* base;
  float norm_eps, hc_eps, cmin, cmax;
  int apply_clamp;
  int iters;
  bf16_t* x_next;        // (T, 4, D)
  bf16_t* y;             // (T, D)
  float* post_out;
  float* comb;
  float* inv_rms;
  float* mixes;
  float* logits;
  float* pre;
  float* pre_ws;         // (T, 4) pre for the y kernel
  int64_t T;
  int D;
};

__device__ __forceinline__ u32x4 lds_read1(uint32_t a) {
  u32x4 v;
  asm volatile("ds_read_b128 %0, %1\n\ts_waitcnt lgkmcnt(0)" : "=v"(v) : "v"(a) : "memory");
  return v;
}

__global__ __launch_bounds__(kPPThreads) void post_pre_fwd_kernel(PostPreArgs a) {
  constexpr int N = kPPN, M = kPPM, MT = kPPMT, L = N * N, TT = kPPTile, S = kPPStages;
  // Stage j's loads have landed once at most V newer vector memory
  // operations are outstanding.  Issued after them: the loads of the S - 2
  // next stages (at least kPPCImin per wave each) and, from stage S - 1 on,
  // the x_next stores of the S - 1 previous stages (kPPCST each; the heads'
  // stores only add).  The first S - 1 stages of a block count loads only.
  constexpr int VM_START = (S - 2) * kPPCImin;
  constexpr int VM_C = (S - 2) * kPPCImin + (S - 1) * kPPCST;
  static_assert(VM_C < 64, "vmcnt range");
  __shared__ u32x4 ring[S * kPPUnits * kWave];
  __shared__ u32x4 gates[3 * kWave];  // h_res rows of the 32 tokens (2 units), h_post (1 unit)
  __shared__ float red_ssq[2][3][16];
  __shared__ float mix_sh[TT][M + 1];
  __shared__ __align__(16) float inv_sh[TT];

  const int tid = threadIdx.x, lane = tid & (kWave - 1);
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int rb = wave & 1, n = wave >> 1;
  const int part_k = n;  // this wave's partial sum of its row block (0 = the reducer)
  const int r = lane & 15, q = lane >> 4;
  const int D = a.D;
  const int64_t K = (int64_t)N * D;
  const int64_t T = a.T;
  const int nst_c = D / kPPCW;
  const int per_tile = nst_c;
  const int64_t ntiles = (T + TT - 1) / TT;
  const int64_t my_tiles = (ntiles - blockIdx.x + gridDim.x - 1) / gridDim.x;
  if (my_tiles <= 0) return;  // uniform over the block
  const int64_t J = my_tiles * per_tile;
  const auto rphi = rows_rsrc(a.phi, (int64_t)M * K * 2);
  const uint32_t gates_lds = lds_addr(gates);

  const int e = tid % L;
  const float a0 = a.alpha[0], a1 = a.alpha[1], a2 = a.alpha[2];
  const float base_l = a.base[2 * N + e];
  const float base_h = e < 2 * N ? a.base[e] : 0.f;

  // Per-lane byte offsets of this wave's contraction-stage units (u = wave +
  // 8i) at d0 = 0 (a stage adds 2*d0) and of its x_next stores; rows >= M of
  // phi are out of range.
  const int nci = wave < kPPUnits - kPPCImin * kPPWaves ? kPPCImax : kPPCImin;
  // DMA lane L of an x / h_out unit: row i = L >> 3 of its half, chunk
  // (L & 7) ^ f(i, g)
  const int di = lane >> 3;
  uint32_t cbase[kPPCImax];
#pragma unroll
  for (int i = 0; i < kPPCImax; ++i) {
    const int u = wave + kPPWaves * i;
    if (u < kUH) {  // x: unit 8rb + 2j + g
      const int ur = u >> 3, uj = (u >> 1) & 3, ug = u & 1;
      const int c = (lane & 7) ^ ((di >> 1) ^ (ug << 2));
      cbase[i] = (uint32_t)((((int64_t)(16 * ur + 8 * ug + di) * N + uj) * D + 8 * c) * 2);
    } else if (u < kUP) {  // h_out: unit 16 + 2rb + g
      const int v = u - kUH, ur = v >> 1, ug = v & 1;
      const int c = (lane & 7) ^ ((di >> 1) ^ (ug << 2));
      cbase[i] = (uint32_t)(((int64_t)(16 * ur + 8 * ug + di) * D + 8 * c) * 2);
    } else {  // phi: unit 20 + 4n + 2h + mt
      const int v = u - kUP, un = v >> 2, uh = (v >> 1) & 1, mt = v & 1;
      cbase[i] = 16 * mt + r < M ? (uint32_t)(((int64_t)(16 * mt + r) * K + (int64_t)un * D + 32 * uh + 8 * q) * 2)
                                 : kBufferOob;
    }
  }
  // x_next stores: instruction 0 writes rows 16rb + (r & 7), instruction 1
  // rows 16rb + 8 + (r & 7); lanes r < 8 write the first 64 bytes of a row
  // segment in instruction 0 and the last 64 in instruction 1, lanes r >= 8
  // the other way round
  const int hi = r >> 3;
  const uint32_t sbase0 = (uint32_t)((((int64_t)(16 * rb + (r & 7)) * N + n) * D + 32 * hi + 8 * q) * 2);
  const uint32_t sbase1 = (uint32_t)((((int64_t)(16 * rb + 8 + (r & 7)) * N + n) * D + 32 * (1 - hi) + 8 * q) * 2);
  // read slots of this lane's x / h_out chunks c = 4h + q of row r
  uint32_t rpos[2];
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    const int c = 4 * h + q, ri = r & 7;
    rpos[h] = (uint32_t)(hi * 1024 + (ri * 8 + (c ^ ((ri >> 1) ^ (hi << 2)))) * 16);
  }

  // ---- loads of stage j (issued S - 1 stages ahead) ------------------------
  int64_t itile = blockIdx.x;
  int is = 0;  // stage of the next issue
  auto issue = [&](int64_t j) {
    const int64_t tb = itile * TT;
    const int nv = (int)(T - tb < TT ? T - tb : TT);
    const uint32_t slot = lds_addr(ring) + (uint32_t)((j % S) * kPPUnits * 1024);
    if (is == 0 && wave == 0) {
      // the tile's gates: h_res rows (64 bytes a token), h_post (16 bytes)
      const auto rg = rows_rsrc(a.h_res + tb * L, (int64_t)nv * L * 4);
#pragma unroll
      for (int u = 0; u < 2; ++u)
        __builtin_amdgcn_raw_ptr_buffer_load_lds(rg, (lds_void_t*)(uintptr_t)(gates_lds + u * 1024), 16,
                                                 (uint32_t)((16 * u + (lane >> 2)) * 64 + (lane & 3) * 16), 0,
                                                 0, 0);
      const auto rp = rows_rsrc(a.h_post + tb * N, (int64_t)nv * N * 4);
      __builtin_amdgcn_raw_ptr_buffer_load_lds(rp, (lds_void_t*)(uintptr_t)(gates_lds + 2048), 16,
                                               lane < TT ? (uint32_t)(lane * 16) : kBufferOob, 0, 0, 0);
    }
    const uint32_t d2 = (uint32_t)(is * kPPCW * 2);
    const auto rx = rows_rsrc(a.x + tb * K, (int64_t)nv * K * 2);
    const auto rh = rows_rsrc(a.h_out + tb * D, (int64_t)nv * D * 2);
#pragma unroll
    for (int i = 0; i < kPPCImax; ++i) {
      if (i < nci) {
        const int u = wave + kPPWaves * i;
        lds_void_t* dst = (lds_void_t*)(uintptr_t)(slot + u * 1024);
        if (u < kUH)
          __builtin_amdgcn_raw_ptr_buffer_load_lds(rx, dst, 16, cbase[i] + d2, 0, 0, 2 /* nt */);
        else if (u < kUP)
          __builtin_amdgcn_raw_ptr_buffer_load_lds(rh, dst, 16, cbase[i] + d2, 0, 0, 2);
        else
          __builtin_amdgcn_raw_ptr_buffer_load_lds(rphi, dst, 16, cbase[i] + d2, 0, 0, 0);
      }
    }
    if (++is == per_tile) {
      is = 0;
      itile += gridDim.x;
    }
  };

  for (int64_t j = 0; j < S - 1 && j < J; ++j) issue(j);

  floatx4 acc[MT];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) acc[mt] = floatx4{0.f, 0.f, 0.f, 0.f};
  float ssq = 0.f;
  float hr[N], hp = 0.f;  // gates of this lane's token for stream n
#pragma unroll
  for (int jj = 0; jj < N; ++jj) hr[jj] = 0.f;
  int64_t ctile = blockIdx.x;
  int cs = 0;  // stage being consumed
  for (int64_t j = 0; j < J; ++j) {
    // this wave's loads of stage j have landed (see VM_C); near the end
    // fewer stages follow it and everything is waited for
    if (j + S - 2 < J) {
      if (j >= S - 1)
        wait_vmcnt<VM_C>();
      else
        wait_vmcnt<VM_START>();
    } else {
      wait_vmcnt<0>();
    }
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
    const uint32_t slot = lds_addr(ring) + (uint32_t)((j % S) * kPPUnits * 1024);
    const int64_t tb = ctile * TT;
    const int nv = (int)(T - tb < TT ? T - tb : TT);

    if (cs < nst_c) {
      // ---- contraction stage --------------------------------------------
      if (j + S - 1 < J) issue(j + S - 1);
      if (cs == 0) {
        // h_res[t][jj][n] (row jj of the token's 64-byte h_res) and h_post[t][n]
        const int tt = 16 * rb + r;
        const uint32_t ga = gates_lds + (tt >> 4) * 1024 + (tt & 15) * 64 + n * 4;
        asm volatile(
            "ds_read_b32 %0, %5\n\t"
            "ds_read_b32 %1, %5 offset:16\n\t"
            "ds_read_b32 %2, %5 offset:32\n\t"
            "ds_read_b32 %3, %5 offset:48\n\t"
            "ds_read_b32 %4, %6\n\t"
            "s_waitcnt lgkmcnt(0)"
            : "=&v"(hr[0]), "=&v"(hr[1]), "=&v"(hr[2]), "=&v"(hr[3]), "=&v"(hp)
            : "v"(ga), "v"(gates_lds + 2048 + tt * 16 + n * 4)
            : "memory");
      }
      // x (streams 0..3) and h_out at columns 64s + 32h + 8c (h = 0, 1) and
      // phi^T of stream n ([h][mt]): one batch of 14 reads and one wait
      u32x4 X0[4], X1[4], H[2], B[4];
      {
        const uint32_t ax = slot + (8 * rb) * 1024;
        const uint32_t ah = slot + (kUH + 2 * rb) * 1024;
        const uint32_t ap = slot + (kUP + 4 * n) * 1024 + lane * 16;
        asm volatile(
            "ds_read_b128 %0, %14\n\t"
            "ds_read_b128 %1, %14 offset:2048\n\t"
            "ds_read_b128 %2, %14 offset:4096\n\t"
            "ds_read_b128 %3, %14 offset:6144\n\t"
            "ds_read_b128 %4, %15\n\t"
            "ds_read_b128 %5, %15 offset:2048\n\t"
            "ds_read_b128 %6, %15 offset:4096\n\t"
            "ds_read_b128 %7, %15 offset:6144\n\t"
            "ds_read_b128 %8, %16\n\t"
            "ds_read_b128 %9, %17\n\t"
            "ds_read_b128 %10, %18\n\t"
            "ds_read_b128 %11, %18 offset:1024\n\t"
            "ds_read_b128 %12, %18 offset:2048\n\t"
            "ds_read_b128 %13, %18 offset:3072\n\t"
            "s_waitcnt lgkmcnt(0)"
            : "=&v"(X0[0]), "=&v"(X0[1]), "=&v"(X0[2]), "=&v"(X0[3]), "=&v"(X1[0]), "=&v"(X1[1]),
              "=&v"(X1[2]), "=&v"(X1[3]), "=&v"(H[0]), "=&v"(H[1]), "=&v"(B[0]), "=&v"(B[1]), "=&v"(B[2]),
              "=&v"(B[3])
            : "v"(ax + rpos[0]), "v"(ax + rpos[1]), "v"(ah + rpos[0]), "v"(ah + rpos[1]), "v"(ap)
            : "memory");
      }
      // x_next for stream n, columns 64s + 32h + 8c..+8 (mhc_post's FMA order)
      u32x4 A[2];
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        float hv[8], xv[N][8];
        Store<bf16_t>::unpack(H[h], hv);
#pragma unroll
        for (int jj = 0; jj < N; ++jj) Store<bf16_t>::unpack(h ? X1[jj] : X0[jj], xv[jj]);
        float o[8];
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          float v = hp * hv[i];
#pragma unroll
          for (int jj = 0; jj < N; ++jj) v = fmaf(hr[jj], xv[jj][i], v);
          o[i] = v;
        }
        A[h] = Store<bf16_t>::pack(o);
      }
      // store x_next as whole 128-byte row segments: lane r takes the second
      // half of lane r ^ 8 (DPP row rotation by 8); rows >= nv fall outside
      // the range and are dropped
      {
        u32x4 S1;
#pragma unroll
        for (int i = 0; i < 4; ++i) S1[i] = (uint32_t)__builtin_amdgcn_mov_dpp((int)A[1][i], kDppRor8, 0xF, 0xF, false);
        const auto rxn = rows_rsrc(a.x_next + tb * K, (int64_t)nv * K * 2);
        const uint32_t d2 = (uint32_t)(cs * kPPCW * 2);
        u32x4 W0, W1;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          W0[i] = hi ? S1[i] : A[0][i];
          W1[i] = hi ? A[0][i] : S1[i];
        }
        __builtin_amdgcn_raw_buffer_store_b128(W0, rxn, sbase0 + d2, 0, 2 /* nt */);
        __builtin_amdgcn_raw_buffer_store_b128(W1, rxn, sbase1 + d2, 0, 2 /* nt */);
      }
      // sum(x_next^2) and the stage's MFMA chain, added to the running sums
      floatx4 part[MT];
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) part[mt] = floatx4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int h = 0; h < 2; ++h) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const float lo = __uint_as_float(A[h][i] << 16), hi2 = __uint_as_float(A[h][i] & 0xffff0000u);
          ssq = fmaf(lo, lo, fmaf(hi2, hi2, ssq));
        }
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) part[mt] = mfma16x16x32(as_bf16x8(A[h]), as_bf16x8(B[2 * h + mt]), part[mt]);
      }
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) acc[mt] += part[mt];

      if (cs == nst_c - 1) {
        // ---- tile's mixes (partials added in a fixed order), heads, Sinkhorn
        // acc: lane (r, c) holds token 16rb + 4c + v, m = 16mt + r; after the
        // shuffles the lanes of row r hold sum(x_next^2) of token 16rb + r
        // over this wave's streams and columns.  The slot of this stage is
        // free once every wave has read it (first barrier) and serves as the
        // exchange buffer: [rb][part_k - 1][mt][lane].
        ssq += __shfl_xor(ssq, 16, kWave);
        ssq += __shfl_xor(ssq, 32, kWave);
        __syncthreads();
        floatx4* xch = reinterpret_cast<floatx4*>(ring + (size_t)(j % S) * kPPUnits * kWave);
        if (part_k != 0) {
#pragma unroll
          for (int mt = 0; mt < MT; ++mt) xch[((rb * 3 + part_k - 1) * MT + mt) * kWave + lane] = acc[mt];
          if (q == 0) red_ssq[rb][part_k - 1][r] = ssq;
        }
        __syncthreads();
        if (part_k == 0) {
          float ssq_t = ssq;
#pragma unroll
          for (int k = 0; k < 3; ++k) {
#pragma unroll
            for (int mt = 0; mt < MT; ++mt) acc[mt] += xch[((rb * 3 + k) * MT + mt) * kWave + lane];
            ssq_t += red_ssq[rb][k][r];
          }
          const float inv_row = 1.0f / sqrtf(ssq_t / (float)K + a.norm_eps);
#pragma unroll
          for (int v = 0; v < 4; ++v) {
            const float inv = __shfl(inv_row, 4 * q + v, kWave);
            const int tt = 16 * rb + 4 * q + v;
#pragma unroll
            for (int mt = 0; mt < MT; ++mt)
              if (16 * mt + r < M) mix_sh[tt][16 * mt + r] = acc[mt][v] * inv;
          }
          if (q == 0) inv_sh[16 * rb + r] = inv_row;
        }
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) acc[mt] = floatx4{0.f, 0.f, 0.f, 0.f};
        ssq = 0.f;
        __syncthreads();
        if (a.mixes) {
          for (int idx = tid; idx < TT * M; idx += kPPThreads) {
            const int tt = idx / M, m = idx - (idx / M) * M;
            if (tt < nv) a.mixes[(tb + tt) * M + m] = mix_sh[tt][m];
          }
        }
        if (a.inv_rms && tid < nv) a.inv_rms[tb + tid] = inv_sh[tid];
        static_assert(kPPThreads / L == TT, "one pass of heads and Sinkhorn");
        {
          const int tt = tid / L;
          const int64_t tok = tb + tt;
          const bool ok = tt < nv;
          const float logit = mix_sh[tt][2 * N + e] * a2 + base_l;
          const float lc = clamp_logit(logit, a.apply_clamp, a.cmin, a.cmax);
          const float c = sinkhorn_fwd<N>(lc, a.hc_eps, a.iters);
          if (ok) {
            a.comb[tok * L + e] = c;
            if (a.logits) a.logits[tok * L + e] = logit;
          }
          if (e < N) {
            const float p = sigmoidf_(mix_sh[tt][e] * a0 + base_h) + a.hc_eps;
            if (ok) {
              a.pre_ws[tok * N + e] = p;
              if (a.pre) a.pre[tok * N + e] = p;
            }
          } else if (e < 2 * N) {
            const float po = 2.0f * sigmoidf_(mix_sh[tt][e] * a1 + base_h);
            if (ok) a.post_out[tok * N + (e - N)] = po;
          }
        }
        __syncthreads();
      }
    }
    if (++cs == per_tile) {
      cs = 0;
      ctile += gridDim.x;
    }
  }
}

bool post_pre_usable(const void* x, const void* h_out, const void* phi, const void* x_next, const void* y,
                     int32_t x_dtype, int32_t phi_dtype, int32_t N, int32_t D) {
  return N == kPPN && x_dtype == MHC_DTYPE_BF16 && phi_dtype == MHC_DTYPE_BF16 && D % kPPCW == 0 &&
         D >= kPPMinD && (int64_t)kPPTile * N * D * 2 < ((int64_t)1 << 31) &&
         (int64_t)kPPM * N * D * 2 < ((int64_t)1 << 31) && aligned16(x) && aligned16(h_out) && aligned16(phi) &&
         aligned16(x_next) && aligned16(y);
}

}  // namespace
}  // namespace mhc

using namespace mhc;

extern "C" size_t mhc_post_pre_fwd_workspace_size(int64_t T, int32_t N, int32_t D, int32_t phi_dtype) {
  return mhc_pre_fwd_workspace_size(T, N, D, phi_dtype);
}

extern "C" int mhc_post_pre_fwd_ex(const void* x, const float* h_res, const void* h_out, const float* h_post,
                                   int32_t x_dtype, const void* phi, int32_t phi_dtype, const float* alpha,
                                   const float* base, float norm_eps, float hc_eps, float clamp_min,
                                   float clamp_max, int32_t iter_times, void* x_next, void* y, float* post_out,
                                   float* comb_frag, float* inv_rms, float* mixes, float* h_res_logits, float* pre,
                                   void* workspace, size_t workspace_bytes, int32_t* status, int64_t T, int32_t N,
                                   int32_t D, void* stream) {
  clear_error();
  if (T < 0 || D <= 0 || N <= 0)
    return set_error(MHC_ERR_INVALID, "mhc_post_pre_fwd: bad shape T=%lld N=%d D=%d", (long long)T, N, D);
  if (int rc = check_tokens(T, "mhc_post_pre_fwd")) return rc;
  if (N != 4 && N != 8)
    return set_error(MHC_ERR_UNSUPPORTED, "mhc_post_pre_fwd: N=%d not supported (4, 8)", N);
  if (T == 0) return MHC_OK;
  if (!x || !h_res || !h_out || !h_post || !phi || !alpha || !base || !x_next || !y || !post_out || !comb_frag)
    return set_error(MHC_ERR_INVALID, "mhc_post_pre_fwd: null pointer");
  if (N == 4 && x_dtype == MHC_DTYPE_BF16 && phi_dtype == MHC_DTYPE_BF16 && workspace) {
    // one pass: x_next formed in the single-pass pre kernel and written once
    bool used = false;
    const int rc = post_pre_fwd_single_pass(x, h_res, h_out, h_post, phi, alpha, base, norm_eps, hc_eps, clamp_min,
                                            clamp_max, iter_times, x_next, y, post_out, comb_frag, inv_rms, mixes,
                                            h_res_logits, pre, workspace, workspace_bytes, status, T, D,
                                            (hipStream_t)stream, &used);
    if (rc || used) return rc;
  }
  if (!post_pre_usable(x, h_out, phi, x_next, y, x_dtype, phi_dtype, N, D) || !workspace ||
      workspace_bytes < fwd_y_ws_bytes(T, N) ||
      pre_fwd_single_pass_applies(x_next, x_dtype, phi, phi_dtype, y, workspace_bytes, T, N, D,
                                  (hipStream_t)stream)) {
    // every other shape, and where the pre forward reads x_next once (its
    // single-pass form: then the post forward plus that move fewer bytes
    // than this kernel plus the y pass): the two operators one after the
    // other
    int rc = mhc_post_fwd(x, h_res, h_out, h_post, x_next, T, N, D, x_dtype, stream);
    if (rc) return rc;
    return mhc_pre_fwd_ex(x_next, x_dtype, phi, phi_dtype, alpha, base, norm_eps, hc_eps, clamp_min, clamp_max,
                          iter_times, y, post_out, comb_frag, inv_rms, mixes, h_res_logits, pre, nullptr, workspace,
                          workspace_bytes, status, T, N, D, stream);
  }
  PostPreArgs a{};
  a.x = static_cast<const bf16_t*>(x);
  a.h_res = h_res;
  a.h_out = static_cast<const bf16_t*>(h_out);
  a.h_post = h_post;
  a.phi = static_cast<const uint16_t*>(phi);
  a.alpha = alpha;
  a.base = base;
  a.norm_eps = norm_eps;
  a.hc_eps = hc_eps;
  a.cmin = clamp_min;
  a.cmax = clamp_max;
  a.apply_clamp = (clamp_min != 0.0f || clamp_max != 0.0f) ? 1 : 0;
  a.iters = iter_times;
  a.x_next = static_cast<bf16_t*>(x_next);
  a.y = static_cast<bf16_t*>(y);
  a.post_out = post_out;
  a.comb = comb_frag;
  a.inv_rms = inv_rms;
  a.mixes = mixes;
  a.logits = h_res_logits;
  a.pre = pre;
  a.pre_ws = static_cast<float*>(workspace);
  a.T = T;
  a.D = D;
  const int64_t ntiles = (T + kPPTile - 1) / kPPTile;
  const int64_t cus = device_cu_count();
  const int64_t grid = ntiles < cus ? ntiles : cus;  // one block per CU (LDS ring)
  hipLaunchKernelGGL(post_pre_fwd_kernel, dim3((unsigned)grid), dim3(kPPThreads), 0, (hipStream_t)stream, a);
  if (int rc = check_launch("post_pre_fwd")) return rc;
  return launch_pre_y_pass(x_next, a.pre_ws, y, T, N, D, (hipStream_t)stream);
}

extern "C" int mhc_post_pre_fwd(const void* x, const float* h_res, const void* h_out, const float* h_post,
                                int32_t x_dtype, const void* phi, int32_t phi_dtype, const float* alpha,
                                const float* base, float norm_eps, float hc_eps, float clamp_min, float clamp_max,
                                int32_t iter_times, void* x_next, void* y, float* post_out, float* comb_frag,
                                float* inv_rms, float* mixes, float* h_res_logits, float* pre, void* workspace,
                                size_t workspace_bytes, int64_t T, int32_t N, int32_t D, void* stream) {
  return mhc_post_pre_fwd_ex(x, h_res, h_out, h_post, x_dtype, phi, phi_dtype, alpha, base, norm_eps, hc_eps,
                             clamp_min, clamp_max, iter_times, x_next, y, post_out, comb_frag, inv_rms, mixes,
                             h_res_logits, pre, workspace, workspace_bytes, nullptr, T, N, D, stream);
}
