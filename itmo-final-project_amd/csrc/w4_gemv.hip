// Decode-shaped W4A16 products (1 <= M <= 16) for gfx950, built to stream
// packed weights at HBM speed.
//
//  * Output column tiles of TN = 16*VEC columns; a lane owns VEC adjacent
//    columns (VEC = 4: one 128-bit load per qweight row; 16 lanes read 256
//    contiguous bytes).
//  * Every wave issues a batch of U*VEC = 16 packed words per lane (4 KB per
//    wave) before it touches any of them, and the next batch is in flight
//    while the current one is dequantized, so each wave keeps up to 8 KB of
//    HBM reads outstanding.
//  * The activation rows of the workgroup's K range and the scales/zeros of its
//    groups are staged once in LDS by the whole workgroup, while the weight
//    loads are in flight; the inner loop then reads only registers and LDS.
//  * Each packed word is dequantized exactly in registers (w4_common.hpp)
//    straight into the B operand of v_mfma_f32_16x16x32_{bf16,f16}; the matrix
//    core performs the K reduction.  Rows m >= M of the A operand repeat row
//    M-1 and their results are discarded.
//  * The NW per-wave partial tiles are summed through LDS in wave order; with
//    a K split (grid.y) the workgroup writes fp32 partials that
//    splitk_reduce_kernel (w4_skinny.hip) sums in split order.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <type_traits>

#include "w4_common.hpp"

namespace w4 {

struct GemvArgs {
  const uint16_t* x;
  int64_t sxm, sxk;
  int M;
  int gshift;
  const uint32_t* qw;
  const uint16_t* sc;
  const uint16_t* ze;
  int64_t N, K;
  uint16_t* y;
  int64_t ldy;
  float* ws;               // fp32 partials [S][M][N] or null
  int64_t steps_per_split; // 32-wide K steps per workgroup (multiple of U)
  int x_contig;
  int sz_per_step;         // group < 32*U: scales change inside a batch
};

template <int VEC>
struct Words {
  uint32_t w[VEC];
};

template <int VEC>
__device__ __forceinline__ void load_words_fast(Words<VEC>& r, const uint32_t* __restrict__ p) {
  if constexpr (VEC == 4) {
    const u32x4 v = *reinterpret_cast<const u32x4*>(p);
    r.w[0] = v[0];
    r.w[1] = v[1];
    r.w[2] = v[2];
    r.w[3] = v[3];
  } else {
    r.w[0] = *p;
  }
}

template <int VEC>
__device__ __forceinline__ void load_words_checked(Words<VEC>& r, const uint32_t* __restrict__ p,
                                                   bool row_ok, int64_t col0, int64_t N) {
#pragma unroll
  for (int j = 0; j < VEC; ++j) r.w[j] = (row_ok && col0 + j < N) ? p[j] : 0u;
}

// LDS carve-up for one workgroup (bytes):
//   xs  : M * KRP uint16    activation rows of the K range (KRP = steps*32, zero padded)
//   szs : NG * TN uint32    (scale | zero << 16) per (group, column)
//   red : NW * M * TN float aliases xs+szs after the main loop
__host__ __device__ inline size_t gemv_lds_bytes(int M, int64_t steps, int64_t ng, int tn, int nw) {
  const size_t a = (size_t)M * (size_t)steps * 32 * 2 + (size_t)ng * tn * 4;
  const size_t b = (size_t)nw * M * tn * 4;
  return a > b ? a : b;
}

template <int DT, int VEC, int U>
__device__ __forceinline__ void gemv_tile(const GemvArgs& a, int64_t n0, int64_t st0, int64_t st1,
                                          int64_t split, unsigned char* smem) {
  typedef typename Act<DT>::frag F;
  constexpr int TN = 16 * VEC;
  const int nw = blockDim.x >> 6;
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wv = tid >> 6;
  const int c = lane & 15, kb = lane >> 4;
  const int64_t N = a.N, K = a.K, K8 = K >> 3;
  const int M = a.M;
  const int64_t col0 = n0 + (int64_t)VEC * c;
  const int64_t kbeg = st0 * 32;
  const int64_t kend = std::min<int64_t>(st1 * 32, K);
  const int KRP = (int)((st1 - st0) * 32);
  const int64_t g0 = kbeg >> a.gshift;
  const int ng = (int)(((kend - 1) >> a.gshift) - g0 + 1);
  uint16_t* xs = reinterpret_cast<uint16_t*>(smem);
  uint32_t* szs = reinterpret_cast<uint32_t*>(smem + (size_t)M * KRP * 2);
  float* red = reinterpret_cast<float*>(smem);
  const bool col_full = (n0 + TN <= N);
  const uint32_t magic = fp16_magic_vgpr();
  const int64_t row_stride4 = 4 * N;  // words between consecutive steps

  // ---- issue this wave's first batch of weight loads
  int64_t s0 = st0 + (int64_t)wv * U;
  const int64_t bstride = (int64_t)nw * U;
  Words<VEC> cur[U];
  auto load_batch = [&](Words<VEC> (&b)[U], int64_t sb) {
    const uint32_t* p = a.qw + (sb * 4 + kb) * N + col0;
    if (col_full && (sb + U) * 4 <= K8 && sb + U <= st1) {
#pragma unroll
      for (int i = 0; i < U; ++i) load_words_fast<VEC>(b[i], p + i * row_stride4);
    } else {
#pragma unroll
      for (int i = 0; i < U; ++i) {
        const bool ok = (sb + i < st1) && ((sb + i) * 4 + kb < K8);
        load_words_checked<VEC>(b[i], p + i * row_stride4, ok, col0, N);
      }
    }
  };
  if (s0 < st1) load_batch(cur, s0);

  // ---- stage activations and scales/zeros in LDS
  {
    const int chunks_per_row = KRP / 8;
    const int total = M * chunks_per_row;
    for (int t = tid; t < total; t += blockDim.x) {
      const int m = t / chunks_per_row;
      const int kk = (t - m * chunks_per_row) * 8;
      const uint16_t* row = a.x + (int64_t)m * a.sxm;
      F f = a.x_contig ? load_x8<DT, true>(row, kbeg + kk, K, a.sxk) : load_x8<DT, false>(row, kbeg + kk, K, a.sxk);
      *reinterpret_cast<F*>(xs + (size_t)m * KRP + kk) = f;
    }
    const int tot2 = ng * TN;
    for (int t = tid; t < tot2; t += blockDim.x) {
      const int gi = t / TN;
      const int nl = t - gi * TN;
      const int64_t n = n0 + nl;
      uint32_t v = 0;
      if (n < N) {
        const int64_t off = (g0 + gi) * N + n;
        v = (uint32_t)a.sc[off] | ((uint32_t)a.ze[off] << 16);
      }
      szs[t] = v;
    }
  }
  __syncthreads();

  f32x4 acc[VEC];
#pragma unroll
  for (int j = 0; j < VEC; ++j) acc[j] = f32x4{0.f, 0.f, 0.f, 0.f};
  const int xrow = (c < M ? c : M - 1) * KRP;

  GroupConst gc[VEC];
  auto compute = [&](const Words<VEC> (&b)[U], int64_t sb, auto checked) {
    constexpr bool CHECK = decltype(checked)::value;
#pragma unroll
    for (int i = 0; i < U; ++i) {
      const int64_t step = sb + i;
      if (CHECK && step >= st1) break;
      const int64_t k8 = step * 4 + kb;
      const bool kok = !CHECK || k8 < K8;
      const int kl = (int)(k8 * 8 - kbeg);
      if (i == 0 || a.sz_per_step) {
        const int gi = (int)(((kok ? k8 : K8 - 1) * 8 >> a.gshift) - g0);
#pragma unroll
        for (int j = 0; j < VEC; ++j) {
          const uint32_t v = szs[gi * TN + VEC * c + j];
          gc[j] = make_group_const((uint16_t)(v & 0xFFFFu), (uint16_t)(v >> 16));
        }
      }
      const F xa = *reinterpret_cast<const F*>(xs + xrow + kl);
#pragma unroll
      for (int j = 0; j < VEC; ++j) {
        F bf = dequant_word<DT>(b[i].w[j], gc[j], magic);
        if (CHECK && !kok) bf = F{};
        acc[j] = Mfma<DT>::m16(xa, bf, acc[j]);
      }
    }
  };

  while (s0 < st1) {
    const int64_t s1 = s0 + bstride;
    Words<VEC> nxt[U];
    if (s1 < st1) load_batch(nxt, s1);
    if ((s0 + U) * 4 <= K8 && s0 + U <= st1)
      compute(cur, s0, std::false_type{});
    else
      compute(cur, s0, std::true_type{});
#pragma unroll
    for (int i = 0; i < U; ++i) cur[i] = nxt[i];
    s0 = s1;
  }

  // ---- cross-wave reduction in wave order
  __syncthreads();
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    const int m = kb * 4 + r;
    if (m < M) {
#pragma unroll
      for (int j = 0; j < VEC; ++j) red[(wv * M + m) * TN + VEC * c + j] = acc[j][r];
    }
  }
  __syncthreads();
  const int total = M * TN;
  for (int idx = tid; idx < total; idx += blockDim.x) {
    const int m = idx / TN;
    const int nl = idx - m * TN;
    const int64_t n = n0 + nl;
    if (n >= N) continue;
    float s = red[m * TN + nl];
    for (int w = 1; w < nw; ++w) s += red[(w * M + m) * TN + nl];
    if (a.ws) {
      a.ws[(split * M + m) * N + n] = s;
    } else {
      a.y[(int64_t)m * a.ldy + n] = float_to_act_bits<DT>(s);
    }
  }
}

template <int DT, int VEC, int U>
__global__ __launch_bounds__(512) __attribute__((amdgpu_waves_per_eu(4, 8))) void gemv_kernel(GemvArgs a) {
  extern __shared__ __attribute__((aligned(16))) unsigned char smem[];
  const int64_t n0 = (int64_t)blockIdx.x * (16 * VEC);
  const int64_t split = blockIdx.y;
  const int64_t steps_total = ((a.K >> 3) + 3) >> 2;
  const int64_t st0 = split * a.steps_per_split;
  const int64_t st1 = std::min<int64_t>(st0 + a.steps_per_split, steps_total);
  gemv_tile<DT, VEC, U>(a, n0, st0, st1, split, smem);
}

struct GemvGroupedArgs {
  GemvArgs prob[W4_MAX_GROUPED];
  int64_t tile_start[W4_MAX_GROUPED + 1];
  int vec[W4_MAX_GROUPED];
  int count;
};

template <int DT>
__global__ __launch_bounds__(512) __attribute__((amdgpu_waves_per_eu(4, 8))) void gemv_grouped_kernel(GemvGroupedArgs g) {
  extern __shared__ __attribute__((aligned(16))) unsigned char smem[];
  const int64_t t = blockIdx.x;
  int p = 0;
#pragma unroll
  for (int i = 1; i < W4_MAX_GROUPED; ++i)
    if (i < g.count && t >= g.tile_start[i]) p = i;
  const GemvArgs& a = g.prob[p];
  const int64_t local = t - g.tile_start[p];
  const int64_t steps_total = ((a.K >> 3) + 3) >> 2;
  if (g.vec[p] == 4)
    gemv_tile<DT, 4, 4>(a, local * 64, 0, steps_total, 0, smem);
  else
    gemv_tile<DT, 1, 16>(a, local * 16, 0, steps_total, 0, smem);
}

}  // namespace w4

// ------------------------------------------------------------------- host side
using namespace w4host;

namespace {

constexpr size_t kGemvLdsBudget = 48 * 1024;

struct GemvPlan {
  int vec, u, nw;
  int64_t tiles, splits, steps_per_split;
  size_t lds, ws;
};

bool gemv_vec4_ok(const void* qw, const void* sc, const void* ze, int64_t N) {
  return (N % 4) == 0 && ((uintptr_t)qw % 16) == 0 && ((uintptr_t)sc % 8) == 0 && ((uintptr_t)ze % 8) == 0;
}

// Static launch table (a pure function of the shape, alignment and CU count).
GemvPlan plan_gemv(int64_t M, int64_t N, int64_t K, int G, bool vec4) {
  GemvPlan p{};
  const int cus = device_cu_count();
  p.vec = vec4 ? 4 : 1;
  if (p.vec == 4 && (N + 63) / 64 < cus / 2) p.vec = 1;  // narrow layer: more, thinner tiles
  p.u = 16 / p.vec;
  const int64_t tn = 16 * p.vec;
  p.tiles = (N + tn - 1) / tn;
  const int64_t steps = ((K / 8) + 3) / 4;
  // K split: for M > 1 aim at >= 2 workgroups per CU; always keep the staged
  // activations within the LDS budget.
  int64_t splits = 1;
  if (M > 1) splits = std::max<int64_t>(1, (2 * cus + p.tiles - 1) / p.tiles);
  const int64_t max_splits = std::max<int64_t>(1, steps / p.u);
  splits = std::min<int64_t>(splits, std::min<int64_t>(max_splits, 16));
  for (;;) {
    int64_t sps = (steps + splits - 1) / splits;
    sps = (sps + p.u - 1) / p.u * p.u;
    const int64_t ng = (std::min<int64_t>(sps * 32, K) + G - 1) / G + 1;
    p.nw = (int)std::min<int64_t>(8, std::max<int64_t>(1, (sps + p.u - 1) / p.u));
    p.lds = w4::gemv_lds_bytes((int)M, sps, ng, (int)tn, p.nw);
    if (p.lds <= kGemvLdsBudget || splits >= steps) {
      p.splits = (steps + sps - 1) / sps;
      p.steps_per_split = sps;
      break;
    }
    ++splits;
  }
  p.ws = p.splits > 1 ? (size_t)p.splits * M * N * sizeof(float) : 0;
  return p;
}

}  // namespace

size_t w4_gemv_workspace_bytes(int64_t M, int64_t N, int64_t K, int G) {
  const size_t a = plan_gemv(M, N, K, G, (N % 4) == 0).ws;
  const size_t b = plan_gemv(M, N, K, G, false).ws;
  return a > b ? a : b;
}

int w4_splitk_reduce_launch(const float* ws, int S, int64_t M, int64_t N, int x_dtype, void* y, int64_t ldy,
                            hipStream_t st);

int w4_gemv_launch(const void* x, int x_dtype, int64_t M, int64_t N, int64_t K, int64_t sxm, int64_t sxk,
                   const int32_t* qw, const uint16_t* sc, const uint16_t* ze, int G, void* y, int64_t ldy,
                   void* ws, size_t ws_bytes, hipStream_t st) {
  const GemvPlan p = plan_gemv(M, N, K, G, gemv_vec4_ok(qw, sc, ze, N));
  if (p.ws > 0 && (ws == nullptr || ws_bytes < p.ws))
    return fail(W4_ERR_WORKSPACE, "w4a16_gemm: workspace of %zu bytes required, %zu given", p.ws,
                ws ? ws_bytes : (size_t)0);
  if (p.lds > kGemvLdsBudget) return fail(W4_ERR_UNSUPPORTED, "w4a16_gemm: decode tile does not fit in LDS");
  w4::GemvArgs a{};
  a.x = static_cast<const uint16_t*>(x);
  a.sxm = sxm;
  a.sxk = sxk;
  a.M = (int)M;
  a.gshift = ilog2(G);
  a.qw = reinterpret_cast<const uint32_t*>(qw);
  a.sc = sc;
  a.ze = ze;
  a.N = N;
  a.K = K;
  a.y = static_cast<uint16_t*>(y);
  a.ldy = ldy;
  a.ws = p.splits > 1 ? static_cast<float*>(ws) : nullptr;
  a.steps_per_split = p.steps_per_split;
  a.x_contig = (sxk == 1) && ((uintptr_t)x % 16 == 0) && (M == 1 || (sxm % 8) == 0);
  a.sz_per_step = (G < 32 * p.u) ? 1 : 0;
  const dim3 grid((unsigned)p.tiles, (unsigned)p.splits);
  const dim3 block(p.nw * 64);
  if (x_dtype == W4_DTYPE_BF16) {
    if (p.vec == 4) hipLaunchKernelGGL((w4::gemv_kernel<W4_DTYPE_BF16, 4, 4>), grid, block, p.lds, st, a);
    else hipLaunchKernelGGL((w4::gemv_kernel<W4_DTYPE_BF16, 1, 16>), grid, block, p.lds, st, a);
  } else {
    if (p.vec == 4) hipLaunchKernelGGL((w4::gemv_kernel<W4_DTYPE_FP16, 4, 4>), grid, block, p.lds, st, a);
    else hipLaunchKernelGGL((w4::gemv_kernel<W4_DTYPE_FP16, 1, 16>), grid, block, p.lds, st, a);
  }
  int rc = check_launch("w4a16_gemm (decode)");
  if (rc != W4_OK || p.splits == 1) return rc;
  return w4_splitk_reduce_launch(static_cast<const float*>(ws), (int)p.splits, M, N, x_dtype, y, ldy, st);
}

// Grouped decode launch; returns W4_ERR_UNSUPPORTED (nothing launched) when
// some problem's activation rows do not fit the LDS budget, so the caller can
// fall back to per-problem launches.
int w4_gemv_grouped_launch(const w4a16_problem* problems, int count, int x_dtype, int64_t M, hipStream_t st) {
  w4::GemvGroupedArgs g{};
  g.count = count;
  int64_t tiles = 0;
  size_t lds = 0;
  const int nw = 8;
  for (int i = 0; i < count; ++i) {
    const w4a16_problem& q = problems[i];
    w4::GemvArgs& a = g.prob[i];
    const int64_t G = q.group_size;
    const bool vec4 = gemv_vec4_ok(q.qweight, q.scales, q.zeros, q.N) && q.K <= 4096;
    g.vec[i] = vec4 ? 4 : 1;
    const int tn = 16 * g.vec[i];
    const int64_t steps = ((q.K / 8) + 3) / 4;
    const size_t need = w4::gemv_lds_bytes((int)M, steps, (q.K + G - 1) / G + 1, tn, nw);
    if (need > kGemvLdsBudget) return W4_ERR_UNSUPPORTED;
    lds = std::max(lds, need);
    a.x = static_cast<const uint16_t*>(q.x);
    a.sxm = q.K;
    a.sxk = 1;
    a.M = (int)M;
    a.gshift = ilog2(G);
    a.qw = reinterpret_cast<const uint32_t*>(q.qweight);
    a.sc = q.scales;
    a.ze = q.zeros;
    a.N = q.N;
    a.K = q.K;
    a.y = static_cast<uint16_t*>(q.y);
    a.ldy = q.N;
    a.ws = nullptr;
    a.steps_per_split = steps;
    a.x_contig = ((uintptr_t)q.x % 16 == 0) && (M == 1 || q.K % 8 == 0);
    a.sz_per_step = (G < 32 * (16 / g.vec[i])) ? 1 : 0;
    g.tile_start[i] = tiles;
    tiles += (q.N + tn - 1) / tn;
  }
  for (int i = count; i <= W4_MAX_GROUPED; ++i) g.tile_start[i] = tiles;
  if (x_dtype == W4_DTYPE_BF16)
    hipLaunchKernelGGL((w4::gemv_grouped_kernel<W4_DTYPE_BF16>), dim3((unsigned)tiles), dim3(nw * 64), lds, st, g);
  else
    hipLaunchKernelGGL((w4::gemv_grouped_kernel<W4_DTYPE_FP16>), dim3((unsigned)tiles), dim3(nw * 64), lds, st, g);
  return check_launch("w4a16_gemm_grouped");
}
