// Prefill W4A16 GEMM (M > 64) for gfx950: y[M, N] = x[M, K] @ W_hat^T.
//
// Tiling (this library's own design; the reference's Triton kernel is
// int4_triton/gemm.py:74-157 with the M > 64 launch at :270-296):
//  * Workgroup tile BM x BN = 128 x 256, K step BK = 64, four waves side by
//    side along N, each owning a 128 x 64 output block computed with
//    v_mfma_f32_32x32x16_{bf16,f16} (4 x 2 blocks of 32 x 32, fp32 accumulate).
//  * The activation tile is staged through LDS (double-buffered, one barrier
//    per K step) because all four waves read it.
//  * The int4 weight never goes through LDS: the MFMA B operand of a lane is
//    8 consecutive k of one column, which is exactly one packed qweight word,
//    so each wave loads its own words (coalesced 128-byte row segments) and
//    dequantizes them in registers straight into the operand, once per
//    workgroup M tile (128 rows share every dequantized value).
//  * The next K step's activation chunks and packed words are loaded into
//    registers while the current step's MFMAs run.
#include <hip/hip_runtime.h>

#include "w4_common.hpp"

namespace w4 {

struct PrefillArgs {
  const uint16_t* x;
  int64_t sxm, sxk;
  int64_t M, N, K;
  const int32_t* qw;
  const uint16_t* sc;
  const uint16_t* ze;
  int gshift;
  int x_contig;
  uint16_t* y;
  int64_t ldy;
  int64_t tiles_n;
};

constexpr int PF_BM = 128;
constexpr int PF_BN = 256;
constexpr int PF_BK = 64;
constexpr int PF_WAVES = 4;
constexpr int PF_XLD = PF_BK + 8;  // padded LDS row (elements)

template <int DT>
__global__ __launch_bounds__(PF_WAVES * 64) void prefill_kernel(PrefillArgs a) {
  typedef typename Act<DT>::frag F;
  __shared__ __attribute__((aligned(16))) uint16_t xs[2][PF_BM * PF_XLD];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wn = tid >> 6;
  const int64_t tile_m = blockIdx.x / a.tiles_n;
  const int64_t tile_n = blockIdx.x % a.tiles_n;
  const int64_t m0 = tile_m * PF_BM;
  const int64_t n0 = tile_n * PF_BN + (int64_t)wn * 64;
  const int64_t K8 = a.K >> 3;
  const int64_t KT = (a.K + PF_BK - 1) / PF_BK;
  const int l32 = lane & 31, lh = lane >> 5;
  const uint32_t magic = fp16_magic_vgpr();
  const bool sz_per_ks = (a.gshift < 6);  // group < BK: scales change inside a K step

  // ---- activation tile loader: 128 rows x 64 k = 1024 chunks of 8 elements.
  u32x4 xr[4];
  auto load_x = [&](int64_t kt) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int id = tid + i * 256;
      const int row = id >> 3;
      const int kc = (id & 7) * 8;
      const int64_t m = m0 + row, k = kt * PF_BK + kc;
      if (m < a.M && k < a.K) {
        const uint16_t* rp = a.x + m * a.sxm;
        F f = a.x_contig ? load_x8<DT, true>(rp, k, a.K, a.sxk) : load_x8<DT, false>(rp, k, a.K, a.sxk);
        xr[i] = __builtin_bit_cast(u32x4, f);
      } else {
        xr[i] = u32x4{0u, 0u, 0u, 0u};
      }
    }
  };
  auto store_x = [&](int buf) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int id = tid + i * 256;
      const int row = id >> 3;
      const int kc = (id & 7) * 8;
      *reinterpret_cast<u32x4*>(&xs[buf][row * PF_XLD + kc]) = xr[i];
    }
  };

  // ---- packed weights of this wave: [ks][nb], k8 = kt*8 + 2*ks + lh,
  // column n0 + nb*32 + l32.
  uint32_t wr[4][2], wn_[4][2];
  uint16_t sr[4][2], zr[4][2], sn[4][2], zn[4][2];
  auto load_w = [&](int64_t kt, uint32_t (&w)[4][2], uint16_t (&s)[4][2], uint16_t (&z)[4][2]) {
#pragma unroll
    for (int nb = 0; nb < 2; ++nb) {
      const int64_t n = n0 + nb * 32 + l32;
      const bool nok = n < a.N;
#pragma unroll
      for (int ks = 0; ks < 4; ++ks) {
        const int64_t k8 = kt * 8 + 2 * ks + lh;
        const bool ok = nok && k8 < K8;
        w[ks][nb] = ok ? (uint32_t)a.qw[k8 * a.N + n] : 0u;
        if (ks == 0 || sz_per_ks) {
          const int64_t kk8 = (k8 < K8) ? k8 : (kt * 8 < K8 ? kt * 8 : 0);
          const int64_t g = (kk8 * 8) >> a.gshift;
          s[ks][nb] = nok ? a.sc[g * a.N + n] : (uint16_t)0;
          z[ks][nb] = nok ? a.ze[g * a.N + n] : (uint16_t)0;
        }
      }
    }
  };

  f32x16 acc[4][2];
#pragma unroll
  for (int mb = 0; mb < 4; ++mb)
#pragma unroll
    for (int nb = 0; nb < 2; ++nb)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[mb][nb][r] = 0.0f;

  load_x(0);
  load_w(0, wr, sr, zr);
  store_x(0);
  __syncthreads();

  for (int64_t kt = 0; kt < KT; ++kt) {
    const int buf = (int)(kt & 1);
    const bool more = kt + 1 < KT;
    if (more) {
      load_x(kt + 1);
      load_w(kt + 1, wn_, sn, zn);
    }
    GroupConst gc[2];
#pragma unroll
    for (int nb = 0; nb < 2; ++nb) gc[nb] = make_group_const(sr[0][nb], zr[0][nb]);
    const uint16_t* xb = xs[buf];
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) {
      F af[4], bf[2];
#pragma unroll
      for (int mb = 0; mb < 4; ++mb) {
        const u32x4 v = *reinterpret_cast<const u32x4*>(&xb[(mb * 32 + l32) * PF_XLD + ks * 16 + lh * 8]);
        af[mb] = __builtin_bit_cast(F, v);
      }
#pragma unroll
      for (int nb = 0; nb < 2; ++nb) {
        if (sz_per_ks && ks > 0) gc[nb] = make_group_const(sr[ks][nb], zr[ks][nb]);
        bf[nb] = dequant_word<DT>(wr[ks][nb], gc[nb], magic);
        const int64_t k8 = kt * 8 + 2 * ks + lh;
        if (k8 >= K8) bf[nb] = F{};
      }
#pragma unroll
      for (int mb = 0; mb < 4; ++mb)
#pragma unroll
        for (int nb = 0; nb < 2; ++nb) acc[mb][nb] = Mfma<DT>::m32(af[mb], bf[nb], acc[mb][nb]);
    }
    if (more) {
      store_x(buf ^ 1);
#pragma unroll
      for (int ks = 0; ks < 4; ++ks)
#pragma unroll
        for (int nb = 0; nb < 2; ++nb) {
          wr[ks][nb] = wn_[ks][nb];
          sr[ks][nb] = sn[ks][nb];
          zr[ks][nb] = zn[ks][nb];
        }
    }
    __syncthreads();
  }

  // ---- epilogue: D[row][col] of a 32x32 block lives in lane (col + 32*h),
  // register r with row = 8*(r/4) + 4*h + (r%4).
#pragma unroll
  for (int mb = 0; mb < 4; ++mb)
#pragma unroll
    for (int nb = 0; nb < 2; ++nb) {
      const int64_t n = n0 + nb * 32 + l32;
      if (n >= a.N) continue;
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int64_t m = m0 + mb * 32 + 8 * (r >> 2) + 4 * lh + (r & 3);
        if (m < a.M) a.y[m * a.ldy + n] = float_to_act_bits<DT>(acc[mb][nb][r]);
      }
    }
}

}  // namespace w4

using namespace w4host;

int w4_prefill_launch(const void* x, int x_dtype, int64_t M, int64_t N, int64_t K, int64_t sxm,
                      int64_t sxk, const int32_t* qw, const uint16_t* sc, const uint16_t* ze, int G,
                      void* y, int64_t ldy, hipStream_t st) {
  w4::PrefillArgs a{};
  a.x = static_cast<const uint16_t*>(x);
  a.sxm = sxm;
  a.sxk = sxk;
  a.M = M;
  a.N = N;
  a.K = K;
  a.qw = qw;
  a.sc = sc;
  a.ze = ze;
  a.gshift = ilog2(G);
  a.x_contig = (sxk == 1) && ((uintptr_t)x % 16 == 0) && (sxm % 8 == 0);
  a.y = static_cast<uint16_t*>(y);
  a.ldy = ldy;
  a.tiles_n = (N + w4::PF_BN - 1) / w4::PF_BN;
  const int64_t tiles_m = (M + w4::PF_BM - 1) / w4::PF_BM;
  const dim3 grid((unsigned)(tiles_m * a.tiles_n));
  const dim3 block(w4::PF_WAVES * 64);
  if (x_dtype == W4_DTYPE_BF16)
    hipLaunchKernelGGL((w4::prefill_kernel<W4_DTYPE_BF16>), grid, block, 0, st, a);
  else
    hipLaunchKernelGGL((w4::prefill_kernel<W4_DTYPE_FP16>), grid, block, 0, st, a);
  return check_launch("w4a16_gemm (prefill)");
}
