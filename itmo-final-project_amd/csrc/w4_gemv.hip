// Decode-shaped W4A16 products (1 <= M <= 16) for gfx950, built to stream
// packed weights at HBM speed while the dequantization keeps pace.
//
//  * Output column tiles of TN = 16*VEC columns; a lane owns VEC adjacent
//    columns (VEC = 4: one 128-bit load per qweight row, 16 lanes read 256
//    contiguous bytes of a row).
//  * Each wave owns a contiguous run of 32-wide K steps and streams it as a
//    double-buffered pipeline of small batches (U steps): the next batch's
//    weights, activation fragments and scales/zeros are in flight while the
//    current batch is dequantized.  Waves never wait on each other until the
//    final reduction, so dequantization overlaps the HBM stream instead of
//    starting after it.
//  * Weights are read with buffer loads: one VGPR offset per lane plus SGPR
//    step offsets, so the inner loop spends no VALU on addressing; tail
//    batches use per-lane offsets, which the hardware range check turns into
//    zeros past the end of qweight.
//  * Each packed word is dequantized exactly in registers (w4_common.hpp)
//    straight into the B operand of v_mfma_f32_16x16x32_{bf16,f16}; the matrix
//    core performs the K reduction.  Rows m >= M of the A operand repeat row
//    M-1 and their results are discarded.
//  * The per-wave partial tiles are summed through LDS in wave order.  A K
//    range split over S workgroups either writes fp32 partials for
//    splitk_reduce_kernel (w4_skinny.hip, separate launch), or, in the grouped
//    launch, is finished by the last workgroup of the tile to arrive: it reads
//    the S partials in split order (a per-tile arrival counter, reset after
//    use, only elects that workgroup), so every bit of the result is fixed.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <type_traits>

#include "w4_common.hpp"

namespace w4 {

struct GemvArgs {
  const uint16_t* x;
  int64_t sxm, sxk;
  const uint32_t* qw;
  const uint16_t* sc;
  const uint16_t* ze;
  uint16_t* y;
  float* ws;               // fp32 partials [S][M][N] or null
  unsigned* counters;      // per-tile arrival counters (in-kernel fixup) or null
  int64_t ldy;
  uint32_t qw_bytes;       // qweight bytes: loads at or past it read 0
  uint32_t sz_bytes;       // scales (= zeros) bytes
  int N, K;
  int M;
  int gshift;              // log2(group size)
  int steps_per_split;     // 32-wide K steps per workgroup
  int splits;
  int x_contig;
};

// Buffer resource word 3 for gfx9-family raw buffers: 32-bit data format.
constexpr int kBufferFlags = 0x00020000;

template <int VEC>
struct WordT;
template <>
struct WordT<4> {
  typedef u32x4 T;
  __device__ __forceinline__ static T load(__amdgpu_buffer_rsrc_t r, uint32_t vo, uint32_t so) {
    return __builtin_amdgcn_raw_buffer_load_b128(r, vo, so, 0);
  }
  __device__ __forceinline__ static uint32_t get(const T& v, int j) { return v[j]; }
};
template <>
struct WordT<1> {
  typedef uint32_t T;
  __device__ __forceinline__ static T load(__amdgpu_buffer_rsrc_t r, uint32_t vo, uint32_t so) {
    return __builtin_amdgcn_raw_buffer_load_b32(r, vo, so, 0);
  }
  __device__ __forceinline__ static uint32_t get(const T& v, int) { return v; }
};

// Scales and zeros of VEC adjacent columns (fp16 bit patterns).
template <int VEC>
struct SZ {
  uint32_t s[VEC > 1 ? VEC / 2 : 1];  // VEC = 4: two packed pairs; VEC = 1: low half
  uint32_t z[VEC > 1 ? VEC / 2 : 1];
  __device__ __forceinline__ uint16_t sj(int j) const {
    return VEC == 1 ? (uint16_t)s[0] : (uint16_t)(s[j >> 1] >> (16 * (j & 1)));
  }
  __device__ __forceinline__ uint16_t zj(int j) const {
    return VEC == 1 ? (uint16_t)z[0] : (uint16_t)(z[j >> 1] >> (16 * (j & 1)));
  }
};

template <int VEC>
__device__ __forceinline__ SZ<VEC> load_sz(__amdgpu_buffer_rsrc_t rs, __amdgpu_buffer_rsrc_t rz, uint32_t off) {
  SZ<VEC> r;
  if constexpr (VEC == 4) {
    const u32x2 a = __builtin_amdgcn_raw_buffer_load_b64(rs, off, 0, 0);
    const u32x2 b = __builtin_amdgcn_raw_buffer_load_b64(rz, off, 0, 0);
    r.s[0] = a[0];
    r.s[1] = a[1];
    r.z[0] = b[0];
    r.z[1] = b[1];
  } else {
    r.s[0] = __builtin_amdgcn_raw_buffer_load_b16(rs, off, 0, 0);
    r.z[0] = __builtin_amdgcn_raw_buffer_load_b16(rz, off, 0, 0);
  }
  return r;
}

template <int DT, int VEC, int U>
struct Batch {
  typename WordT<VEC>::T w[U];
  typename Act<DT>::frag xa[U];
  SZ<VEC> sz[U];
};

// Byte offset that every buffer access treats as out of range (reads 0, no
// memory traffic): used for batches past the end of a wave's run, so that the
// load sequence of the pipelined loop is unconditional.
constexpr uint32_t kOutOfRange = 0x80000000u;

// One workgroup: column tile at n0 (tile index tile_id), K steps [st0, st1)
// of split `split`.  Writes y (DT) when the problem is not split, otherwise
// fp32 partials, finished in-kernel when arrival counters are given.
// SZS: scales/zeros loaded per step and per lane (group < 32*U, or any
// group when batches are not U-aligned); otherwise once per batch.
// Requires x rows dense (unit k stride, 16-byte aligned rows).
template <int DT, int VEC, int U, bool SZS>
__device__ __forceinline__ void gemv_tile(const GemvArgs& a, int n0, int st0, int st1, int split, int tile_id,
                                          float* red) {
  typedef typename Act<DT>::frag F;
  constexpr int TN = 16 * VEC;
  const int nw = blockDim.x >> 6;
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wv = tid >> 6;
  const int c = lane & 15, kb = lane >> 4;
  const int N = a.N, K = a.K, K8 = K >> 3;
  const int M = a.M;
  const int col0 = n0 + VEC * c;
  const uint32_t magic = fp16_magic_vgpr();
  const __amdgpu_buffer_rsrc_t rq =
      __builtin_amdgcn_make_buffer_rsrc((void*)a.qw, (short)0, (int)a.qw_bytes, kBufferFlags);
  const __amdgpu_buffer_rsrc_t rs =
      __builtin_amdgcn_make_buffer_rsrc((void*)a.sc, (short)0, (int)a.sz_bytes, kBufferFlags);
  const __amdgpu_buffer_rsrc_t rz =
      __builtin_amdgcn_make_buffer_rsrc((void*)a.ze, (short)0, (int)a.sz_bytes, kBufferFlags);
  const uint32_t x_bytes = (uint32_t)(((int64_t)(M - 1) * a.sxm + K) * 2);
  const __amdgpu_buffer_rsrc_t rx =
      __builtin_amdgcn_make_buffer_rsrc((void*)a.x, (short)0, (int)x_bytes, kBufferFlags);
  const uint32_t step_bytes = 16u * (uint32_t)N;  // four qweight rows
  const uint32_t lane_off = ((uint32_t)kb * (uint32_t)N + (uint32_t)col0) * 4u;
  const uint32_t x_lane = (uint32_t)((int64_t)(c < M ? c : M - 1) * a.sxm * 2) + (uint32_t)kb * 16u;

  // This wave's contiguous run of steps, a multiple of U long (the launcher
  // keeps st0 a multiple of 8, so batches are U-aligned).
  const int nsteps = st1 - st0;
  const int per_wave = ((nsteps + nw - 1) / nw + U - 1) / U * U;
  const int w_begin = st0 + min(nsteps, wv * per_wave);
  const int w_end = st0 + min(nsteps, (wv + 1) * per_wave);

  // All loads of one batch, unconditionally; a batch at or past w_end reads
  // out-of-range offsets (zeros, no traffic).
  auto load_batch = [&](Batch<DT, VEC, U>& b, int sb) {
    const bool live = sb < w_end;
#pragma unroll
    for (int i = 0; i < U; ++i) {
      if (SZS || i == 0) {
        const int k8 = min((sb + i) * 4 + kb, K8 - 1);
        const uint32_t g = (uint32_t)((k8 * 8) >> a.gshift);
        const uint32_t off = live ? (g * (uint32_t)N + (uint32_t)col0) * 2u : kOutOfRange;
        b.sz[i] = load_sz<VEC>(rs, rz, off);
      }
    }
    const uint32_t vo = live ? (uint32_t)sb * step_bytes + lane_off : kOutOfRange;
    const uint32_t xo = live ? x_lane + (uint32_t)sb * 64u : kOutOfRange;
#pragma unroll
    for (int i = 0; i < U; ++i) {
      b.w[i] = WordT<VEC>::load(rq, vo + (uint32_t)i * step_bytes, 0u);
      b.xa[i] = __builtin_bit_cast(F, __builtin_amdgcn_raw_buffer_load_b128(rx, xo + (uint32_t)i * 64u, 0, 0));
    }
  };

  f32x4 acc[VEC];
#pragma unroll
  for (int j = 0; j < VEC; ++j) acc[j] = f32x4{0.f, 0.f, 0.f, 0.f};
  GroupConst gc[VEC];
  int cur_g = -1;

  auto compute = [&](const Batch<DT, VEC, U>& b, int sb, auto checked) {
    constexpr bool CHECK = decltype(checked)::value;
#pragma unroll
    for (int i = 0; i < U; ++i) {
      const int step = sb + i;
      if (CHECK && step >= w_end) break;
      const int k8 = step * 4 + kb;
      if (SZS) {
#pragma unroll
        for (int j = 0; j < VEC; ++j) gc[j] = make_group_const(b.sz[i].sj(j), b.sz[i].zj(j));
      } else if (i == 0) {
        // constants change at group boundaries only: keep the previous
        // batch's when this batch continues the same group
        const int g = (step * 32) >> a.gshift;
        if (g != cur_g) {
#pragma unroll
          for (int j = 0; j < VEC; ++j) gc[j] = make_group_const(b.sz[0].sj(j), b.sz[0].zj(j));
          cur_g = g;
        }
      }
      F xa = b.xa[i];
      if (CHECK && k8 >= K8) xa = F{};  // past K: the row's next elements are not ours
#pragma unroll
      for (int j = 0; j < VEC; ++j) {
        F bf = dequant_word<DT>(WordT<VEC>::get(b.w[i], j), gc[j], magic);
        if (CHECK && k8 >= K8) bf = F{};
        acc[j] = Mfma<DT>::m16(xa, bf, acc[j]);
      }
    }
  };
  auto run = [&](const Batch<DT, VEC, U>& b, int sb) {
    if (sb >= w_end) return;
    if ((sb + U) * 4 <= K8 && sb + U <= w_end)
      compute(b, sb, std::false_type{});
    else
      compute(b, sb, std::true_type{});
  };

  // Double-buffered pipeline: the loads of batch t+1 are in flight while
  // batch t is computed.
  Batch<DT, VEC, U> ba, bb;
  int s0 = w_begin;
  load_batch(ba, s0);
  for (; s0 < w_end; s0 += 2 * U) {
    load_batch(bb, s0 + U);
    run(ba, s0);
    load_batch(ba, s0 + 2 * U);
    run(bb, s0 + U);
  }

  // ---- cross-wave reduction in wave order
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
  const bool split_out = a.splits > 1;
  const bool fixup = split_out && a.counters != nullptr;
  for (int idx = tid; idx < total; idx += blockDim.x) {
    const int m = idx / TN;
    const int nl = idx - m * TN;
    const int n = n0 + nl;
    if (n >= N) continue;
    float s = red[m * TN + nl];
    for (int w = 1; w < nw; ++w) s += red[(w * M + m) * TN + nl];
    if (!split_out)
      a.y[(int64_t)m * a.ldy + n] = float_to_act_bits<DT>(s);
    else
      a.ws[((int64_t)split * M + m) * N + n] = s;
  }
  if (!fixup) return;

  // ---- in-kernel split-K fixup: the last workgroup of this tile to arrive
  // sums the partials of all splits in split order.  The barrier makes every
  // wave's partial stores complete in this XCD's L2; one lane then releases
  // them at device scope (L2 write-back) before bumping the tile counter, and
  // only the finishing workgroup acquires (dropping its XCD's stale copies of
  // the reused workspace), so the cache-wide operations run once per
  // workgroup and once per tile.
  __shared__ unsigned arrived;
  __syncthreads();
  if (tid == 0) {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "agent");
    const unsigned old =
        __hip_atomic_fetch_add(&a.counters[tile_id], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    if (old == (unsigned)(a.splits - 1)) __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
    arrived = old;
  }
  __syncthreads();
  if (arrived != (unsigned)(a.splits - 1)) return;
  for (int idx = tid; idx < total; idx += blockDim.x) {
    const int m = idx / TN;
    const int nl = idx - m * TN;
    const int n = n0 + nl;
    if (n >= N) continue;
    const float* p = a.ws + (int64_t)m * N + n;
    float s = __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    for (int sp = 1; sp < a.splits; ++sp)
      s += __hip_atomic_load(p + (int64_t)sp * M * N, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    a.y[(int64_t)m * a.ldy + n] = float_to_act_bits<DT>(s);
  }
  if (tid == 0) __hip_atomic_store(&a.counters[tile_id], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

template <int DT, int VEC, int U>
__global__ __launch_bounds__(512) void gemv_kernel(GemvArgs a) {
  extern __shared__ __attribute__((aligned(16))) float red_smem[];
  const int n0 = blockIdx.x * (16 * VEC);
  const int split = blockIdx.y;
  const int steps_total = ((a.K >> 3) + 3) >> 2;
  const int st0 = split * a.steps_per_split;
  const int st1 = min(st0 + a.steps_per_split, steps_total);
  if (a.gshift < 5 + __builtin_ctz(U))
    gemv_tile<DT, VEC, U, true>(a, n0, st0, st1, split, blockIdx.x, red_smem);
  else
    gemv_tile<DT, VEC, U, false>(a, n0, st0, st1, split, blockIdx.x, red_smem);
}

// Grouped launch: problem p owns workgroups [tile_start[p], tile_start[p+1]),
// split-major inside a problem; vec[p] selects the column tiling.
struct GemvGroupedArgs {
  GemvArgs prob[W4_MAX_GROUPED];
  int tile_start[W4_MAX_GROUPED + 1];
  int tiles_n[W4_MAX_GROUPED];
  int vec[W4_MAX_GROUPED];
  int count;
};

template <int DT>
__global__ __launch_bounds__(512) void gemv_grouped_kernel(GemvGroupedArgs g) {
  extern __shared__ __attribute__((aligned(16))) float red_smem[];
  const int t = blockIdx.x;
  int p = 0;
#pragma unroll
  for (int i = 1; i < W4_MAX_GROUPED; ++i)
    if (i < g.count && t >= g.tile_start[i]) p = i;
  const GemvArgs& a = g.prob[p];
  const int local = t - g.tile_start[p];
  const int tn = g.tiles_n[p];
  const int split = local / tn;
  const int tile = local - split * tn;
  const int steps_total = ((a.K >> 3) + 3) >> 2;
  const int st0 = split * a.steps_per_split;
  const int st1 = min(st0 + a.steps_per_split, steps_total);
  const bool szs = a.gshift < 6;  // group < 32*U (U = 2)
  if (g.vec[p] == 4) {
    if (szs)
      gemv_tile<DT, 4, 2, true>(a, tile * 64, st0, st1, split, tile, red_smem);
    else
      gemv_tile<DT, 4, 2, false>(a, tile * 64, st0, st1, split, tile, red_smem);
  } else {
    if (szs)
      gemv_tile<DT, 1, 2, true>(a, tile * 16, st0, st1, split, tile, red_smem);
    else
      gemv_tile<DT, 1, 2, false>(a, tile * 16, st0, st1, split, tile, red_smem);
  }
}

}  // namespace w4

// ------------------------------------------------------------------- host side
using namespace w4host;

namespace {

struct GemvPlan {
  int vec, nw;
  int tiles, splits, steps_per_split;
  size_t lds, ws;
};

bool gemv_vec4_ok(const void* qw, const void* sc, const void* ze, int64_t N) {
  return (N % 4) == 0 && ((uintptr_t)qw % 16) == 0 && ((uintptr_t)sc % 8) == 0 && ((uintptr_t)ze % 8) == 0;
}

// Work per grouped workgroup: 64 K steps (2048 k) of a 64-column tile = 64 KB
// of packed weights, eight waves of 8 steps each.
constexpr int kStepsPerWG = 64;
constexpr int kWaves = 8;

// Static launch table (a pure function of the shape, alignment and CU count).
GemvPlan plan_gemv(int64_t M, int64_t N, int64_t K, bool vec4) {
  GemvPlan p{};
  const int cus = device_cu_count();
  p.vec = vec4 ? 4 : 1;
  const int64_t tn = 16 * p.vec;
  p.tiles = (int)((N + tn - 1) / tn);
  const int64_t steps = ((K / 8) + 3) / 4;
  int64_t splits = 1;
  if (M > 1) {
    // split-K toward >= 2 workgroups per CU (fp32 partials + reduce kernel)
    splits = std::max<int64_t>(1, (2 * cus + p.tiles - 1) / p.tiles);
    splits = std::min<int64_t>(splits, std::max<int64_t>(1, steps / 16));
    splits = std::min<int64_t>(splits, 16);
  }
  const int64_t sps = ((steps + splits - 1) / splits + 7) / 8 * 8;
  p.splits = (int)((steps + sps - 1) / sps);
  p.steps_per_split = (int)sps;
  p.nw = (int)std::min<int64_t>(kWaves, std::max<int64_t>(1, sps / 4));
  p.lds = (size_t)p.nw * M * tn * sizeof(float);
  p.ws = p.splits > 1 ? (size_t)p.splits * M * N * sizeof(float) : 0;
  return p;
}

void fill_args(w4::GemvArgs& a, const void* x, int64_t sxm, int64_t sxk, int64_t M, int64_t N, int64_t K,
               const int32_t* qw, const uint16_t* sc, const uint16_t* ze, int G, void* y, int64_t ldy) {
  a.x = static_cast<const uint16_t*>(x);
  a.sxm = sxm;
  a.sxk = sxk;
  a.qw = reinterpret_cast<const uint32_t*>(qw);
  a.sc = sc;
  a.ze = ze;
  a.y = static_cast<uint16_t*>(y);
  a.ws = nullptr;
  a.counters = nullptr;
  a.ldy = ldy;
  a.qw_bytes = (uint32_t)((K / 8) * N * 4);
  a.sz_bytes = (uint32_t)((K / G) * N * 2);
  a.N = (int)N;
  a.K = (int)K;
  a.M = (int)M;
  a.gshift = ilog2(G);
  a.splits = 1;
  a.x_contig = (sxk == 1) && ((uintptr_t)x % 16 == 0) && (M == 1 || (sxm % 8) == 0);
}

bool fits_32bit(int64_t N, int64_t K) {
  return N < (1LL << 30) && K < (1LL << 30) && (K / 8) * N * 4 < (1LL << 31);
}

template <int DT>
void launch_gemv(const GemvPlan& p, dim3 grid, dim3 block, hipStream_t st, const w4::GemvArgs& a) {
  if (p.vec == 4)
    hipLaunchKernelGGL((w4::gemv_kernel<DT, 4, 2>), grid, block, p.lds, st, a);
  else
    hipLaunchKernelGGL((w4::gemv_kernel<DT, 1, 2>), grid, block, p.lds, st, a);
}

// Grouped plan: every problem is cut into workgroups of one 64-column tile (16
// columns when the 128-bit path is not possible) x kStepsPerWG K steps;
// longer K is split and finished in-kernel.  Workspace layout:
// [counters, zero on entry and on exit][pad to 256 B][fp32 partials].
struct GroupedPlan {
  w4::GemvGroupedArgs g;
  int wgs;
  size_t lds;
  size_t counter_bytes;  // padded to 256
  size_t float_count;
  size_t off_float[W4_MAX_GROUPED];
  size_t off_counter[W4_MAX_GROUPED];
};

bool plan_grouped(const w4a16_problem* problems, int count, int64_t M, GroupedPlan& gp) {
  gp = GroupedPlan{};
  gp.g.count = count;
  int wgs = 0;
  size_t floats = 0, counters = 0;
  for (int i = 0; i < count; ++i) {
    const w4a16_problem& q = problems[i];
    if (!fits_32bit(q.N, q.K) || ((uintptr_t)q.x % 16) != 0 || M * q.K * 2 >= (1LL << 31)) return false;
    const bool vec4 = gemv_vec4_ok(q.qweight, q.scales, q.zeros, q.N);
    const int vec = vec4 ? 4 : 1;
    const int tn = 16 * vec;
    const int tiles = (int)((q.N + tn - 1) / tn);
    const int64_t steps = ((q.K / 8) + 3) / 4;
    const int64_t per = kStepsPerWG;
    const int splits = (int)((steps + per - 1) / per);
    w4::GemvArgs& a = gp.g.prob[i];
    fill_args(a, q.x, q.K, 1, M, q.N, q.K, q.qweight, q.scales, q.zeros, q.group_size, q.y, q.N);
    a.splits = splits;
    a.steps_per_split = (int)(((steps + splits - 1) / splits + 7) / 8 * 8);
    gp.g.vec[i] = vec;
    gp.g.tiles_n[i] = tiles;
    gp.g.tile_start[i] = wgs;
    if (splits > 1) {
      gp.off_float[i] = floats;
      gp.off_counter[i] = counters;
      floats += (size_t)splits * M * q.N;
      counters += (size_t)tiles;
    }
    wgs += tiles * splits;
  }
  for (int i = count; i <= W4_MAX_GROUPED; ++i) gp.g.tile_start[i] = wgs;
  gp.wgs = wgs;
  gp.lds = (size_t)kWaves * M * 64 * sizeof(float);
  gp.counter_bytes = counters * sizeof(unsigned);
  gp.float_count = floats;
  return gp.counter_bytes <= W4_WORKSPACE_COUNTER_BYTES;
}

}  // namespace

// Scratch bytes (past the workspace's counter area) of the single-problem
// paths.  M == 1 runs as a one-problem grouped launch (partials finished
// in-kernel); 2 <= M <= 16 writes fp32 partials for the reduce kernel.
size_t w4_decode_workspace_bytes(const w4a16_problem* problems, const int64_t* sxm, int count, int64_t M,
                                 const int64_t* mrows = nullptr);

size_t w4_gemv_workspace_bytes(int64_t M, int64_t N, int64_t K, int G) {
  if (M == 1) {
    // the decode kernel's K split (aligned operands; counter area only) or the
    // grouped gemv kernel's split partials (groups below 32): room for either
    static char aligned_stand_in[256] __attribute__((aligned(256)));
    w4a16_problem q{aligned_stand_in, reinterpret_cast<const int32_t*>(aligned_stand_in),
                    reinterpret_cast<const uint16_t*>(aligned_stand_in),
                    reinterpret_cast<const uint16_t*>(aligned_stand_in), aligned_stand_in, N, K, G, 0};
    const int64_t sx = K;
    // the decode kernel's split needs the counter area only: one byte of
    // scratch makes the caller's size query non-zero
    const size_t dec = w4_decode_workspace_bytes(&q, &sx, 1, 1) > 0 ? 1 : 0;
    GroupedPlan gp;
    if (!plan_grouped(&q, 1, 1, gp)) return dec;
    const size_t grp = gp.float_count * sizeof(float);
    return grp > dec ? grp : dec;
  }
  const size_t a = plan_gemv(M, N, K, (N % 4) == 0).ws;
  const size_t b = plan_gemv(M, N, K, false).ws;
  return a > b ? a : b;
}

int w4_gemv_grouped_launch(const w4a16_problem* problems, int count, int x_dtype, int64_t M,
                           unsigned* counters, void* scratch, size_t scratch_bytes, hipStream_t st);

int w4_splitk_reduce_launch(const float* ws, int S, int64_t M, int64_t N, int x_dtype, void* y, int64_t ldy,
                            hipStream_t st);

int w4_skinny_launch(const void* x, int x_dtype, int64_t M, int64_t N, int64_t K, int64_t sxm, int64_t sxk,
                     const int32_t* qw, const uint16_t* sc, const uint16_t* ze, int G, void* y, int64_t ldy,
                     void* ws, size_t ws_bytes, hipStream_t st);

int w4_decode_launch(const w4a16_problem* problems, const int64_t* sxm, const int64_t* ldy, int count,
                     int x_dtype, int64_t M, unsigned* counters, void* scratch, size_t scratch_bytes,
                     hipStream_t st, const int64_t* mrows = nullptr);

int w4_gemv_launch(const void* x, int x_dtype, int64_t M, int64_t N, int64_t K, int64_t sxm, int64_t sxk,
                   const int32_t* qw, const uint16_t* sc, const uint16_t* ze, int G, void* y, int64_t ldy,
                   unsigned* counters, void* ws, size_t ws_bytes, hipStream_t st) {
  // The decode kernel reads dense, 16-byte aligned activation rows; other
  // layouts (strided views) take the generic skinny kernel.
  const bool x_dense = sxk == 1 && ((uintptr_t)x % 16) == 0 && (M == 1 || (sxm % 8) == 0) &&
                       (int64_t)M * sxm * 2 < (1LL << 31);
  if (!x_dense)
    return w4_skinny_launch(x, x_dtype, M, N, K, sxm, sxk, qw, sc, ze, G, y, ldy, ws, ws_bytes, st);
  if (!fits_32bit(N, K)) return fail(W4_ERR_UNSUPPORTED, "w4a16_gemm: qweight larger than 2 GiB");
  {
    // group size >= 32: factored single-launch decode kernel (w4_decode.hip)
    const w4a16_problem q{x, qw, sc, ze, y, N, K, G, 0};
    const int rc = w4_decode_launch(&q, &sxm, &ldy, 1, x_dtype, M, counters, ws, ws_bytes, st);
    if (rc != W4_ERR_UNSUPPORTED) return rc;
  }
  // M == 1: the grouped kernel with its in-kernel split fixup.  Without a
  // workspace it refuses (W4_ERR_WORKSPACE, nothing launched) rather than
  // taking another route, so the summation order is a function of the shape.
  if (M == 1 && sxk == 1 && ldy == N) {
    w4a16_problem q{x, qw, sc, ze, y, N, K, G, 0};
    const int rc = w4_gemv_grouped_launch(&q, 1, x_dtype, 1, counters, ws, ws_bytes, st);
    if (rc != W4_ERR_UNSUPPORTED) return rc;
    clear_error();  // too many tiles for the counter area: unsplit launch below
  }
  const GemvPlan p = plan_gemv(M, N, K, gemv_vec4_ok(qw, sc, ze, N));
  if (p.ws > 0 && (ws == nullptr || ws_bytes < p.ws))
    return fail(W4_ERR_WORKSPACE, "w4a16_gemm: workspace of %zu bytes required, %zu given", p.ws,
                ws ? ws_bytes : (size_t)0);
  w4::GemvArgs a{};
  fill_args(a, x, sxm, sxk, M, N, K, qw, sc, ze, G, y, ldy);
  a.splits = p.splits;
  a.ws = p.splits > 1 ? static_cast<float*>(ws) : nullptr;
  a.steps_per_split = p.steps_per_split;
  const dim3 grid((unsigned)p.tiles, (unsigned)p.splits);
  const dim3 block(p.nw * 64);
  if (x_dtype == W4_DTYPE_BF16)
    launch_gemv<W4_DTYPE_BF16>(p, grid, block, st, a);
  else
    launch_gemv<W4_DTYPE_FP16>(p, grid, block, st, a);
  int rc = check_launch("w4a16_gemm (decode)");
  if (rc != W4_OK || p.splits == 1) return rc;
  return w4_splitk_reduce_launch(static_cast<const float*>(ws), p.splits, M, N, x_dtype, y, ldy, st);
}

// Scratch bytes (past the counter area) of a grouped launch; -1 if the
// problems cannot be launched as one group.
int64_t w4_gemv_grouped_scratch_bytes(const w4a16_problem* problems, int count, int64_t M) {
  GroupedPlan gp;
  if (!plan_grouped(problems, count, M, gp)) return -1;
  return (int64_t)(gp.float_count * sizeof(float));
}

// Grouped decode launch.  Returns W4_ERR_UNSUPPORTED (nothing launched, no
// error message) if a problem is too large for 32-bit offsets or the tiles
// exceed the counter area.
int w4_gemv_grouped_launch(const w4a16_problem* problems, int count, int x_dtype, int64_t M,
                           unsigned* counters, void* scratch, size_t scratch_bytes, hipStream_t st) {
  if (count >= 1 && count <= W4_MAX_GROUPED) {
    int64_t sxm[W4_MAX_GROUPED];
    for (int i = 0; i < count; ++i) sxm[i] = problems[i].K;
    const int rc = w4_decode_launch(problems, sxm, nullptr, count, x_dtype, M, counters, scratch, scratch_bytes, st);
    if (rc != W4_ERR_UNSUPPORTED) return rc;
  }
  GroupedPlan gp;
  if (!plan_grouped(problems, count, M, gp)) return W4_ERR_UNSUPPORTED;
  if (gp.counter_bytes > 0) {
    const size_t need = gp.float_count * sizeof(float);
    if (counters == nullptr || scratch == nullptr || scratch_bytes < need)
      return fail(W4_ERR_WORKSPACE, "w4a16 decode: workspace of %zu bytes required",
                  (size_t)W4_WORKSPACE_COUNTER_BYTES + need);
    unsigned* cbase = counters;
    float* fbase = static_cast<float*>(scratch);
    for (int i = 0; i < count; ++i) {
      w4::GemvArgs& a = gp.g.prob[i];
      if (a.splits > 1) {
        a.ws = fbase + gp.off_float[i];
        a.counters = cbase + gp.off_counter[i];
      }
    }
  }
  if (x_dtype == W4_DTYPE_BF16)
    hipLaunchKernelGGL((w4::gemv_grouped_kernel<W4_DTYPE_BF16>), dim3((unsigned)gp.wgs), dim3(kWaves * 64), gp.lds,
                       st, gp.g);
  else
    hipLaunchKernelGGL((w4::gemv_grouped_kernel<W4_DTYPE_FP16>), dim3((unsigned)gp.wgs), dim3(kWaves * 64), gp.lds,
                       st, gp.g);
  return check_launch("w4a16_gemm_grouped");
}
