// Skinny W4A16 products (17 <= M <= 64) for gfx950: the split-K path with fp32
// partials plus the fixed-order reduce kernel (also used by the decode path).
//
// Work decomposition (this library's own; the reference's Triton kernels are
// int4_triton/gemm.py:74-157, :171-182, :185-220):
//  * The output is cut into column tiles of TN = 16*VEC columns.  A lane owns
//    VEC adjacent columns and reads their packed words of one K/8 row with a
//    single 4*VEC-byte load (VEC = 4: a 128-bit load; 16 lanes cover 256
//    contiguous bytes of a qweight row).
//  * The product itself runs on the matrix cores: one packed word is exactly
//    the 8-element k-slice a lane supplies to v_mfma_f32_16x16x32_{bf16,f16},
//    so each word is dequantized in registers straight into an MFMA operand
//    (no LDS staging, no re-layout).  For M == 1 fifteen of the sixteen MFMA
//    rows are padding; the matrix cores have ~10x the needed throughput, and
//    the cross-lane K reduction happens inside the MFMA instead of in
//    shuffles.
//  * A workgroup of NW waves owns one column tile and a contiguous K range;
//    waves take interleaved batches of U 32-wide K steps, with the next batch's
//    loads in flight while the current batch is dequantized and multiplied.
//    The NW per-wave partial tiles are summed through LDS in wave order.
//  * If the K range is split over S workgroups (grid.y), each writes fp32
//    partials [S][M][N] and w4_splitk_reduce_kernel sums them in split order.
//  Every summation order is fixed by (M, N, K, G, CU count), so results are
//  bit-identical from run to run.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <type_traits>

#include "w4_common.hpp"

namespace w4 {

struct SkinnyArgs {
  const uint16_t* x;
  int64_t sxm, sxk;
  int64_t M;
  const int32_t* qw;
  const uint16_t* sc;
  const uint16_t* ze;
  int64_t N, K;
  int gshift;      // log2(group size)
  int x_contig;    // x rows are dense and 16-byte aligned
  int sz_per_step; // group size < 32*U: scales change inside a batch
  void* y;
  int64_t ldy;
  float* ws;       // fp32 partials [S][M][N] (split-K) or null
  int64_t steps_per_split;
};

template <int MB>
struct SkinnyCfg {
  static constexpr int U = (MB <= 1) ? 4 : 2;  // K steps (of 32) per batch
};

template <int VEC>
struct WordVec;
template <>
struct WordVec<4> {
  typedef u32x4 T;
};
template <>
struct WordVec<1> {
  typedef uint32_t T;
};

template <int VEC>
__device__ __forceinline__ uint32_t word_at(const typename WordVec<VEC>::T& v, int j) {
  if constexpr (VEC == 1) {
    return v;
  } else {
    return v[j];
  }
}

// Load the VEC packed words of row k8, columns col0 .. col0+VEC-1 (0 past N).
template <int VEC>
__device__ __forceinline__ typename WordVec<VEC>::T load_words(const int32_t* __restrict__ qw,
                                                              int64_t k8, int64_t col0,
                                                              int64_t N) {
  typedef typename WordVec<VEC>::T T;
  const uint32_t* p = reinterpret_cast<const uint32_t*>(qw) + k8 * N + col0;
  if constexpr (VEC == 1) {
    return col0 < N ? *p : 0u;
  } else {
    if (col0 + VEC <= N) return *reinterpret_cast<const T*>(p);
    T v;
#pragma unroll
    for (int j = 0; j < VEC; ++j) v[j] = (col0 + j < N) ? p[j] : 0u;
    return v;
  }
}

// Scales and zeros of group g for the VEC columns (packed fp16 pairs).
template <int VEC>
struct SZ {
  uint16_t s[VEC], z[VEC];
};

template <int VEC>
__device__ __forceinline__ SZ<VEC> load_sz(const uint16_t* __restrict__ sc,
                                           const uint16_t* __restrict__ ze, int64_t g,
                                           int64_t col0, int64_t N) {
  SZ<VEC> r;
  const int64_t base = g * N + col0;
  if constexpr (VEC == 4) {
    if (col0 + 4 <= N) {
      const u32x2 s2 = *reinterpret_cast<const u32x2*>(sc + base);
      const u32x2 z2 = *reinterpret_cast<const u32x2*>(ze + base);
      r.s[0] = (uint16_t)s2[0];
      r.s[1] = (uint16_t)(s2[0] >> 16);
      r.s[2] = (uint16_t)s2[1];
      r.s[3] = (uint16_t)(s2[1] >> 16);
      r.z[0] = (uint16_t)z2[0];
      r.z[1] = (uint16_t)(z2[0] >> 16);
      r.z[2] = (uint16_t)z2[1];
      r.z[3] = (uint16_t)(z2[1] >> 16);
      return r;
    }
  }
#pragma unroll
  for (int j = 0; j < VEC; ++j) {
    const bool ok = col0 + j < N;
    r.s[j] = ok ? sc[base + j] : (uint16_t)0;
    r.z[j] = ok ? ze[base + j] : (uint16_t)0;
  }
  return r;
}

template <int DT, int VEC, int MB>
struct Batch {
  static constexpr int U = SkinnyCfg<MB>::U;
  typename WordVec<VEC>::T w[U];
  SZ<VEC> sz[U];  // only [0] used when scales are constant over the batch
  typename Act<DT>::frag xa[U][MB];
  bool valid[U];
};

// Issue every global load of one batch (U steps starting at step s0).
template <int DT, int VEC, int MB>
__device__ __forceinline__ void load_batch(const SkinnyArgs& a, Batch<DT, VEC, MB>& b, int64_t s0,
                                           int64_t st_end, int64_t K8, int kb, int c,
                                           int64_t col0) {
  constexpr int U = SkinnyCfg<MB>::U;
#pragma unroll
  for (int i = 0; i < U; ++i) {
    const int64_t k8 = (s0 + i) * 4 + kb;
    b.valid[i] = (s0 + i < st_end) && (k8 < K8);
    if (b.valid[i]) {
      b.w[i] = load_words<VEC>(a.qw, k8, col0, a.N);
    } else {
      b.w[i] = typename WordVec<VEC>::T{};
    }
    if (a.sz_per_step || i == 0) {
      const int64_t kk8 = b.valid[i] ? k8 : ((s0 * 4 < K8) ? s0 * 4 : 0);
      b.sz[i] = load_sz<VEC>(a.sc, a.ze, (kk8 * 8) >> a.gshift, col0, a.N);
    }
#pragma unroll
    for (int mb = 0; mb < MB; ++mb) {
      const int64_t m = mb * 16 + c;
      typedef typename Act<DT>::frag F;
      if (b.valid[i] && m < a.M) {
        const uint16_t* row = a.x + m * a.sxm;
        b.xa[i][mb] = a.x_contig ? load_x8<DT, true>(row, k8 * 8, a.K, a.sxk)
                                 : load_x8<DT, false>(row, k8 * 8, a.K, a.sxk);
      } else {
        b.xa[i][mb] = F{};
      }
    }
  }
}

template <int DT, int VEC, int MB>
__device__ __forceinline__ void compute_batch(const SkinnyArgs& a, const Batch<DT, VEC, MB>& b,
                                              f32x4 (&acc)[MB][VEC], uint32_t magic) {
  constexpr int U = SkinnyCfg<MB>::U;
  typedef typename Act<DT>::frag F;
  GroupConst gc[VEC];
#pragma unroll
  for (int j = 0; j < VEC; ++j) gc[j] = make_group_const(b.sz[0].s[j], b.sz[0].z[j]);
#pragma unroll
  for (int i = 0; i < U; ++i) {
    if (a.sz_per_step && i > 0) {
#pragma unroll
      for (int j = 0; j < VEC; ++j) gc[j] = make_group_const(b.sz[i].s[j], b.sz[i].z[j]);
    }
#pragma unroll
    for (int j = 0; j < VEC; ++j) {
      F bf = dequant_word<DT>(word_at<VEC>(b.w[i], j), gc[j], magic);
      if (!b.valid[i]) bf = F{};
#pragma unroll
      for (int mb = 0; mb < MB; ++mb) acc[mb][j] = Mfma<DT>::m16(b.xa[i][mb], bf, acc[mb][j]);
    }
  }
}

// One workgroup: column tile starting at n0, K steps [st_begin, st_end).
// Writes the tile's sum over its K range to y (dtype DT) or, if `partial`,
// to ws[split][m][n] in fp32.
template <int DT, int VEC, int MB>
__device__ __forceinline__ void skinny_tile(const SkinnyArgs& a, int64_t n0, int64_t st_begin,
                                            int64_t st_end, bool partial, int64_t split,
                                            float* red) {
  constexpr int U = SkinnyCfg<MB>::U;
  constexpr int TN = 16 * VEC;
  const int nw = blockDim.x >> 6;
  const int lane = threadIdx.x & 63;
  const int wv = threadIdx.x >> 6;
  const int c = lane & 15, kb = lane >> 4;
  const int64_t col0 = n0 + (int64_t)VEC * c;
  const int64_t K8 = a.K >> 3;
  const uint32_t magic = fp16_magic_vgpr();

  f32x4 acc[MB][VEC];
#pragma unroll
  for (int mb = 0; mb < MB; ++mb)
#pragma unroll
    for (int j = 0; j < VEC; ++j) acc[mb][j] = f32x4{0.f, 0.f, 0.f, 0.f};

  int64_t s0 = st_begin + (int64_t)wv * U;
  const int64_t stride = (int64_t)nw * U;
  if (s0 < st_end) {
    Batch<DT, VEC, MB> cur;
    load_batch<DT, VEC, MB>(a, cur, s0, st_end, K8, kb, c, col0);
    while (true) {
      const int64_t s1 = s0 + stride;
      if (s1 < st_end) {
        Batch<DT, VEC, MB> nxt;
        load_batch<DT, VEC, MB>(a, nxt, s1, st_end, K8, kb, c, col0);
        compute_batch<DT, VEC, MB>(a, cur, acc, magic);
        cur = nxt;
        s0 = s1;
      } else {
        compute_batch<DT, VEC, MB>(a, cur, acc, magic);
        break;
      }
    }
  }

  // Cross-wave reduction: red[w][m][TN] for m < M, summed in wave order.
  const int64_t M = a.M;
#pragma unroll
  for (int mb = 0; mb < MB; ++mb)
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int64_t m = mb * 16 + kb * 4 + r;
      if (m < M) {
#pragma unroll
        for (int j = 0; j < VEC; ++j) red[((int64_t)wv * M + m) * TN + VEC * c + j] = acc[mb][j][r];
      }
    }
  __syncthreads();
  const int64_t total = M * TN;
  for (int64_t idx = threadIdx.x; idx < total; idx += blockDim.x) {
    const int64_t m = idx / TN;
    const int nl = (int)(idx % TN);
    const int64_t n = n0 + nl;
    if (n >= a.N) continue;
    float s = red[m * TN + nl];
    for (int w = 1; w < nw; ++w) s += red[((int64_t)w * M + m) * TN + nl];
    if (partial) {
      a.ws[(split * M + m) * a.N + n] = s;
    } else {
      reinterpret_cast<uint16_t*>(a.y)[m * a.ldy + n] = float_to_act_bits<DT>(s);
    }
  }
}

template <int DT, int VEC, int MB>
__global__ __launch_bounds__(512) void skinny_kernel(SkinnyArgs a) {
  extern __shared__ float red[];
  const int64_t n0 = (int64_t)blockIdx.x * (16 * VEC);
  const int64_t split = blockIdx.y;
  const int64_t steps_total = ((a.K >> 3) + 3) >> 2;
  const int64_t st_begin = split * a.steps_per_split;
  int64_t st_end = st_begin + a.steps_per_split;
  if (st_end > steps_total) st_end = steps_total;
  skinny_tile<DT, VEC, MB>(a, n0, st_begin, st_end, a.ws != nullptr, split, red);
}

// y[m][n] = sum_{s < S} ws[s][m][n] in split order (int4_triton/gemm.py:171-182
// is the reference's fixed-order reduce).
// Fixed-order split-K reduce: y = sum over s = 0..S-1 of partial s, in split
// order, cast once.  A thread owns U chunks of VEC consecutive elements of the
// [M, N] result (chunk u of workgroup b: b * 256 U + 256 u + thread, so each
// load instruction of a workgroup covers 256 consecutive chunks) and issues
// the loads of all its chunks and splits (buffer loads; splits S..SMAX-1 take
// an out-of-range offset and are not added) before the first add, so the
// kernel costs one memory latency instead of S.
constexpr int kReduceMaxSplits = 16;
template <int DT, int VEC, int SMAX, int U>
__global__ __launch_bounds__(256) void splitk_reduce_kernel(const float* __restrict__ ws, int S,
                                                            int64_t M, int64_t N,
                                                            uint16_t* __restrict__ y, int64_t ldy) {
  typedef typename std::conditional<VEC == 4, f32x4, float>::type V;
  const int64_t MN = M * N;
  const __amdgpu_buffer_rsrc_t rw =
      __builtin_amdgcn_make_buffer_rsrc((void*)ws, (short)0, (int)((uint64_t)S * MN * 4u), 0x00020000);
  int64_t e[U];
  V v[U][SMAX];
#pragma unroll
  for (int u = 0; u < U; ++u) {
    e[u] = ((int64_t)blockIdx.x * 256 * U + 256 * u + threadIdx.x) * VEC;
    const bool in = e[u] < MN;
#pragma unroll
    for (int i = 0; i < SMAX; ++i) {
      const uint32_t off = (in && i < S) ? (uint32_t)(((int64_t)i * MN + e[u]) * 4) : 0x80000000u;
      if constexpr (VEC == 4)
        v[u][i] = __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(rw, off, 0, 0));
      else
        v[u][i] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rw, off, 0, 0));
    }
  }
#pragma unroll
  for (int u = 0; u < U; ++u) {
    if (e[u] >= MN) continue;
    V t = v[u][0];
#pragma unroll
    for (int i = 1; i < SMAX; ++i)
      if (i < S) t += v[u][i];
    const int64_t m = e[u] / N, n = e[u] - m * N;
    if constexpr (VEC == 4) {
      const uint32_t lo = (uint32_t)float_to_act_bits<DT>(t[0]) | ((uint32_t)float_to_act_bits<DT>(t[1]) << 16);
      const uint32_t hi = (uint32_t)float_to_act_bits<DT>(t[2]) | ((uint32_t)float_to_act_bits<DT>(t[3]) << 16);
      *reinterpret_cast<u32x2*>(y + m * ldy + n) = u32x2{lo, hi};
    } else {
      y[m * ldy + n] = float_to_act_bits<DT>(t);
    }
  }
}

}  // namespace w4

// ------------------------------------------------------------------- host side
using namespace w4host;

namespace {

struct SkinnyPlan {
  int vec;          // 4 or 1
  int mb;           // ceil(M/16)
  int nw;           // waves per workgroup
  int64_t tiles;    // column tiles
  int64_t splits;   // K splits (grid.y)
  int64_t steps_per_split;
  size_t lds_bytes;
  size_t ws_bytes;
};

int u_for_mb(int mb) { return mb <= 1 ? 4 : 2; }

// Static launch table: a pure function of (M, N, K, G, CU count, alignment).
SkinnyPlan plan_skinny(int64_t M, int64_t N, int64_t K, bool vec4_ok) {
  SkinnyPlan p{};
  p.mb = (int)((M + 15) / 16);
  p.vec = vec4_ok ? 4 : 1;
  // M == 1 has no split-K (one launch, no partials): give narrow layers more
  // workgroups with 16-column tiles instead.
  if (M == 1 && p.vec == 4 && (N + 63) / 64 < device_cu_count() / 2) p.vec = 1;
  const int U = u_for_mb(p.mb);
  p.nw = (p.mb <= 1) ? 8 : 4;
  const int64_t tn = 16 * p.vec;
  p.tiles = (N + tn - 1) / tn;
  const int64_t steps_total = ((K / 8) + 3) / 4;
  // Aim for >= 2 workgroups per CU.  Each split keeps >= nw*U steps (every
  // wave gets a full batch) and a multiple of U steps (batches stay aligned
  // to 32*U-wide K windows, so scales are constant inside a batch when
  // G >= 32*U).
  const int64_t target = 2LL * device_cu_count();
  int64_t splits = 1;
  if (M > 1) {
    const int64_t max_splits = std::max<int64_t>(1, steps_total / ((int64_t)p.nw * U));
    splits = std::min<int64_t>(max_splits, std::max<int64_t>(1, (target + p.tiles - 1) / p.tiles));
    splits = std::min<int64_t>(splits, 16);
  }
  int64_t sps = (steps_total + splits - 1) / splits;
  sps = ((sps + U - 1) / U) * U;
  splits = (steps_total + sps - 1) / sps;
  p.splits = splits;
  p.steps_per_split = sps;
  p.lds_bytes = (size_t)p.nw * (size_t)M * (size_t)tn * sizeof(float);
  p.ws_bytes = splits > 1 ? (size_t)splits * (size_t)M * (size_t)N * sizeof(float) : 0;
  return p;
}

template <int DT, int VEC>
void launch_skinny_mb(int mb, dim3 grid, dim3 block, size_t lds, hipStream_t st,
                      const w4::SkinnyArgs& a) {
  switch (mb) {
    case 1: hipLaunchKernelGGL((w4::skinny_kernel<DT, VEC, 1>), grid, block, lds, st, a); break;
    case 2: hipLaunchKernelGGL((w4::skinny_kernel<DT, VEC, 2>), grid, block, lds, st, a); break;
    case 3: hipLaunchKernelGGL((w4::skinny_kernel<DT, VEC, 3>), grid, block, lds, st, a); break;
    default: hipLaunchKernelGGL((w4::skinny_kernel<DT, VEC, 4>), grid, block, lds, st, a); break;
  }
}

}  // namespace

int w4_splitk_reduce_launch(const float* ws, int S, int64_t M, int64_t N, int x_dtype, void* y, int64_t ldy,
                            hipStream_t st);

// Called by w4a16_gemm for 17 <= M <= 64 (validation already done there).
size_t w4_skinny_workspace_bytes(int64_t M, int64_t N, int64_t K, bool vec4_ok) {
  return plan_skinny(M, N, K, vec4_ok).ws_bytes;
}

bool w4_skinny_vec4_ok(const void* qweight, const void* scales, const void* zeros, int64_t N) {
  return (N % 4) == 0 && ((uintptr_t)qweight % 16) == 0 && ((uintptr_t)scales % 8) == 0 &&
         ((uintptr_t)zeros % 8) == 0;
}

int w4_skinny_launch(const void* x, int x_dtype, int64_t M, int64_t N, int64_t K, int64_t sxm,
                     int64_t sxk, const int32_t* qw, const uint16_t* sc, const uint16_t* ze, int G,
                     void* y, int64_t ldy, void* ws, size_t ws_bytes, hipStream_t st) {
  const bool vec4 = w4_skinny_vec4_ok(qw, sc, ze, N);
  const SkinnyPlan p = plan_skinny(M, N, K, vec4);
  if (p.ws_bytes > 0 && (ws == nullptr || ws_bytes < p.ws_bytes))
    return fail(W4_ERR_WORKSPACE, "w4a16_gemm: workspace of %zu bytes required, %zu given", p.ws_bytes,
                ws ? ws_bytes : (size_t)0);
  if (p.lds_bytes > 64 * 1024) return fail(W4_ERR_UNSUPPORTED, "w4a16_gemm: skinny tile too large");
  w4::SkinnyArgs a{};
  a.x = static_cast<const uint16_t*>(x);
  a.sxm = sxm;
  a.sxk = sxk;
  a.M = M;
  a.qw = qw;
  a.sc = sc;
  a.ze = ze;
  a.N = N;
  a.K = K;
  a.gshift = ilog2(G);
  a.x_contig = (sxk == 1) && ((uintptr_t)x % 16 == 0) && (M == 1 || (sxm % 8) == 0);
  a.sz_per_step = (G < 32 * u_for_mb(p.mb)) ? 1 : 0;
  a.y = y;
  a.ldy = ldy;
  a.ws = p.splits > 1 ? static_cast<float*>(ws) : nullptr;
  a.steps_per_split = p.steps_per_split;
  const dim3 grid((unsigned)p.tiles, (unsigned)p.splits);
  const dim3 block(p.nw * 64);
  if (x_dtype == W4_DTYPE_BF16) {
    if (p.vec == 4) launch_skinny_mb<W4_DTYPE_BF16, 4>(p.mb, grid, block, p.lds_bytes, st, a);
    else launch_skinny_mb<W4_DTYPE_BF16, 1>(p.mb, grid, block, p.lds_bytes, st, a);
  } else {
    if (p.vec == 4) launch_skinny_mb<W4_DTYPE_FP16, 4>(p.mb, grid, block, p.lds_bytes, st, a);
    else launch_skinny_mb<W4_DTYPE_FP16, 1>(p.mb, grid, block, p.lds_bytes, st, a);
  }
  int rc = check_launch("w4a16_gemm (skinny)");
  if (rc != W4_OK || p.splits == 1) return rc;
  return w4_splitk_reduce_launch(static_cast<const float*>(ws), (int)p.splits, M, N, x_dtype, y, ldy, st);
}

template <int DT, int VEC, int SMAX, int U>
static void reduce_go(const float* ws, int S, int64_t M, int64_t N, uint16_t* y, int64_t ldy, hipStream_t st) {
  const int64_t chunks = (M * N + VEC - 1) / VEC;
  const dim3 grid((unsigned)((chunks + 256 * U - 1) / (256 * U)));
  hipLaunchKernelGGL((w4::splitk_reduce_kernel<DT, VEC, SMAX, U>), grid, dim3(256), 0, st, ws, S, M, N, y, ldy);
}

// Loads per thread stay at 8-16: more elements per thread for few splits.
template <int DT>
static void reduce_launch_dt(bool v4, const float* ws, int S, int64_t M, int64_t N, uint16_t* y, int64_t ldy,
                             hipStream_t st) {
  if (!v4) {
    if (S <= 4) reduce_go<DT, 1, 4, 4>(ws, S, M, N, y, ldy, st);
    else reduce_go<DT, 1, 16, 1>(ws, S, M, N, y, ldy, st);
    return;
  }
  if (S <= 2) reduce_go<DT, 4, 2, 4>(ws, S, M, N, y, ldy, st);
  else if (S <= 4) reduce_go<DT, 4, 4, 2>(ws, S, M, N, y, ldy, st);
  else if (S <= 8) reduce_go<DT, 4, 8, 1>(ws, S, M, N, y, ldy, st);
  else reduce_go<DT, 4, 16, 1>(ws, S, M, N, y, ldy, st);
}

int w4_splitk_reduce_launch(const float* ws, int S, int64_t M, int64_t N, int x_dtype, void* y, int64_t ldy,
                            hipStream_t st) {
  const int64_t MN = M * N;
  if (S < 1 || S > w4::kReduceMaxSplits || (uint64_t)S * (uint64_t)MN * 4u >= (1ull << 31))
    return fail(W4_ERR_UNSUPPORTED, "w4a16_gemm: split-K reduce of %d x %lld partials unsupported", S,
                (long long)MN);
  const bool v4 = N % 4 == 0 && ldy % 4 == 0 && (uintptr_t)y % 8 == 0;
  uint16_t* yy = static_cast<uint16_t*>(y);
  if (x_dtype == W4_DTYPE_BF16)
    reduce_launch_dt<W4_DTYPE_BF16>(v4, ws, S, M, N, yy, ldy, st);
  else
    reduce_launch_dt<W4_DTYPE_FP16>(v4, ws, S, M, N, yy, ldy, st);
  return check_launch("w4a16_gemm (split-K reduce)");
}
