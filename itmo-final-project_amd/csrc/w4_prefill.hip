// Prefill W4A16 GEMM (M > 64) for gfx950: y[M, N] = x[M, K] @ W_hat^T.
//
// Kernels in this file (this library's own design; the reference's Triton
// kernel is int4_triton/gemm.py:74-157 with the M > 64 launch at :270-296):
//  * pf3_kernel: the main path (dense 16-byte aligned rows, K % 64 == 0);
//    128 / 64 / 32-row tiles of 64 columns per wave, activations through an
//    LDS ring, each wave's packed words dequantized in registers, cost-model
//    split-K (below).
//  * pf5_kernel: products with about one tile per CU; the weight tile is
//    dequantized once per workgroup into LDS (below).
//  * pf2_kernel: pf3's tiling for K % 64 != 0.
//  * prefill_kernel: strided or unaligned activations, described next.
//
// prefill_kernel:
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

#include <algorithm>

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

// ---------------------------------------------------------------------------
// pf2_kernel: dense-row prefill (the common case).
//
//  * 128-row tiles; NW waves side by side along N, each owning a 128 x 64
//    output block (4 x 2 blocks of v_mfma_f32_32x32x16, 128 accumulators a
//    lane).  Waves never share columns, so every weight is dequantized once
//    per 128 rows and the dequantization VALU work is about half the MFMA
//    time; registers stay within 256 a lane so two waves share each SIMD and
//    one wave's dequantization overlaps the other's matrix work.
//  * Packed weights: one 64-bit buffer load gives a lane two adjacent
//    columns of one k8 row (32 lanes read a 256-byte row segment); block nb of
//    the wave holds the columns of parity nb, so the B operand of a lane is
//    one packed word, dequantized exactly in registers (w4_common.hpp).
//  * Activations: 128 x 64 bf16/fp16 tile per K step through double-buffered
//    LDS (rows padded to 72 elements), read as MFMA A fragments.
//  * Split-K (small M): split s covers K steps [s*T, (s+1)*T) and writes fp32
//    partials [S][M][N], summed in split order by splitk_reduce_kernel; one
//    split writes y directly.
//  * Loads for step t+1 are issued (activations first) before step t is
//    computed; registers ping-pong between two sets, so no copy waits.
struct Pf2Args {
  const uint16_t* x;
  const uint32_t* qw;
  const uint16_t* sc;
  const uint16_t* ze;
  uint16_t* y;
  float* ws;
  int64_t sxm, ldy;
  uint32_t x_bytes, qw_bytes, sz_bytes;
  int M, N, K, gshift;
  int tiles_n, tiles_mn, kt_per_split;
  int y16;  // pf3: y rows 16-byte aligned and N % 8 == 0 (LDS-staged 16-byte output stores)
  // pf5: K cut into ks ranges over as many workgroups (workgroup t: range
  // t / tiles_mn of tile t % tiles_mn), finished by the last to arrive
  // (per-tile arrival counters in cnt, partial tiles in ws); pf3's two-split
  // finish uses cnt and ws the same way
  int ks;
  unsigned* cnt;
};
constexpr int kMaxPf5Split = 4;

constexpr int PF2_BM = 128;
constexpr int PF2_BK = 64;
constexpr int PF2_XLD = PF2_BK + 8;

template <int DT, int NW, bool SZK>
__global__ __launch_bounds__(NW * 64) __attribute__((amdgpu_waves_per_eu(2))) void pf2_kernel(Pf2Args a) {
  typedef typename Act<DT>::frag F;
  constexpr int NT = NW * 64;
  constexpr int XCH = PF2_BM * PF2_BK / 8 / NT;  // 16-byte activation chunks per thread per step
  constexpr int NSZ = SZK ? 4 : 1;                // scale/zero loads per step (per ks when group < 64)
  __shared__ __attribute__((aligned(16))) uint16_t xs[2][PF2_BM * PF2_XLD];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wn = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int l32 = lane & 31, lh = lane >> 5;
  const int t = blockIdx.x;
  const int split = t / a.tiles_mn;
  const int tmn = t - split * a.tiles_mn;
  const int tile_m = tmn / a.tiles_n;
  const int tile_n = tmn - tile_m * a.tiles_n;
  const int m0 = tile_m * PF2_BM;
  const int n0w = (tile_n * NW + wn) * 64;
  const int N = a.N;
  const int KT = (a.K + PF2_BK - 1) / PF2_BK;
  const int kt0 = split * a.kt_per_split;
  const int kt1 = min(kt0 + a.kt_per_split, KT);

  const __amdgpu_buffer_rsrc_t rx = __builtin_amdgcn_make_buffer_rsrc((void*)a.x, (short)0, (int)a.x_bytes, 0x00020000);
  const __amdgpu_buffer_rsrc_t rq = __builtin_amdgcn_make_buffer_rsrc((void*)a.qw, (short)0, (int)a.qw_bytes, 0x00020000);
  const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc((void*)a.sc, (short)0, (int)a.sz_bytes, 0x00020000);
  const __amdgpu_buffer_rsrc_t rz = __builtin_amdgcn_make_buffer_rsrc((void*)a.ze, (short)0, (int)a.sz_bytes, 0x00020000);
  constexpr uint32_t OOB = 0x80000000u;

  // activation chunk c = tid + i*NT: row c / 8, k offset (c % 8) * 8
  uint32_t x_row_off[XCH];
  int x_kc[XCH];
#pragma unroll
  for (int i = 0; i < XCH; ++i) {
    const int c = tid + i * NT;
    const int m = m0 + (c >> 3);
    x_kc[i] = (c & 7) * 8;
    x_row_off[i] = m < a.M ? (uint32_t)((int64_t)m * a.sxm * 2) : OOB;
  }
  const uint32_t w_lane = ((uint32_t)lh * (uint32_t)N + (uint32_t)(n0w + 2 * l32)) * 4u;
  const uint32_t sz_col = (uint32_t)(n0w + 2 * l32) * 2u;
  const uint32_t magic = fp16_magic_vgpr();

  struct Stage {
    u32x4 x[XCH];
    u32x2 w[4];
    uint32_t s[NSZ], z[NSZ];
  };
  // Out-of-range offsets are OR-ed masks (bit 31), never selects between
  // offsets, so no load ends up behind a branch.
  auto load = [&](Stage& st, int kt) {
    const uint32_t lmask = kt < kt1 ? 0u : OOB;  // scalar
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int i = 0; i < XCH; ++i) {
      const int k = kt * PF2_BK + x_kc[i];
      const uint32_t kmask = (uint32_t)((a.K - 1 - k) >> 31) & OOB;  // k >= K (rows are dense)
      st.x[i] = __builtin_amdgcn_raw_buffer_load_b128(rx, (x_row_off[i] + (uint32_t)k * 2u) | kmask | lmask, 0, 0);
    }
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int j = 0; j < NSZ; ++j) {
      const uint32_t g = (uint32_t)((kt * PF2_BK + (SZK ? j * 16 + lh * 8 : 0)) >> a.gshift);
      const uint32_t off = (g * (uint32_t)N * 2u + sz_col) | lmask;
      st.s[j] = __builtin_amdgcn_raw_buffer_load_b32(rs, off, 0, 0);
      st.z[j] = __builtin_amdgcn_raw_buffer_load_b32(rz, off, 0, 0);
    }
    const uint32_t wo = ((uint32_t)kt * 8u * (uint32_t)N * 4u + w_lane) | lmask;
#pragma unroll
    for (int ks = 0; ks < 4; ++ks)
      st.w[ks] = __builtin_amdgcn_raw_buffer_load_b64(rq, wo + (uint32_t)ks * 2u * (uint32_t)N * 4u, 0, 0);
    __builtin_amdgcn_sched_barrier(0);
  };
  auto store_x = [&](const Stage& st, int buf) {
#pragma unroll
    for (int i = 0; i < XCH; ++i) {
      const int c = tid + i * NT;
      *reinterpret_cast<u32x4*>(&xs[buf][(c >> 3) * PF2_XLD + x_kc[i]]) = st.x[i];
    }
  };

  f32x16 acc[4][2];
#pragma unroll
  for (int mb = 0; mb < 4; ++mb)
#pragma unroll
    for (int nb = 0; nb < 2; ++nb)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[mb][nb][r] = 0.0f;

  auto compute = [&](const Stage& st, int buf) {
    const uint16_t* xb = xs[buf];
    GroupConst gc[2];
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) {
      if (ks == 0 || SZK) {
        const int j = SZK ? ks : 0;
#pragma unroll
        for (int nb = 0; nb < 2; ++nb)
          gc[nb] = make_group_const((uint16_t)(st.s[j] >> (16 * nb)), (uint16_t)(st.z[j] >> (16 * nb)));
      }
      F af[4], bf[2];
#pragma unroll
      for (int mb = 0; mb < 4; ++mb)
        af[mb] = __builtin_bit_cast(F, *reinterpret_cast<const u32x4*>(&xb[(mb * 32 + l32) * PF2_XLD + ks * 16 + lh * 8]));
#pragma unroll
      for (int nb = 0; nb < 2; ++nb) bf[nb] = dequant_word<DT>(st.w[ks][nb], gc[nb], magic);
#pragma unroll
      for (int mb = 0; mb < 4; ++mb)
#pragma unroll
        for (int nb = 0; nb < 2; ++nb) acc[mb][nb] = Mfma<DT>::m32(af[mb], bf[nb], acc[mb][nb]);
    }
  };

  // Two register stages ping-pong; step t is computed from LDS buffer t & 1.
  Stage sa, sb;
  load(sa, kt0);
  store_x(sa, 0);
  load(sb, kt0 + 1);
  __syncthreads();
  for (int kt = kt0; kt < kt1; kt += 2) {
    compute(sa, 0);
    if (kt + 1 < kt1) store_x(sb, 1);
    load(sa, kt + 2);
    __syncthreads();
    if (kt + 1 < kt1) compute(sb, 1);
    store_x(sa, 0);
    load(sb, kt + 3);
    __syncthreads();
  }

  // epilogue: D[row][col] of a 32x32 block in lane (col + 32*h), register r,
  // row = 8*(r/4) + 4*h + (r%4); column n0w + 2*col + nb
  const int n = n0w + 2 * l32;
  if (n < N) {
#pragma unroll
    for (int mb = 0; mb < 4; ++mb)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int m = m0 + mb * 32 + 8 * (r >> 2) + 4 * lh + (r & 3);
        if (m >= a.M) continue;
        if (a.ws != nullptr) {
          float2 v;
          v.x = acc[mb][0][r];
          v.y = acc[mb][1][r];
          *reinterpret_cast<float2*>(a.ws + ((int64_t)split * a.M + m) * N + n) = v;
        } else {
          const uint32_t v = (uint32_t)float_to_act_bits<DT>(acc[mb][0][r]) |
                             ((uint32_t)float_to_act_bits<DT>(acc[mb][1][r]) << 16);
          *reinterpret_cast<uint32_t*>(a.y + (int64_t)m * a.ldy + n) = v;
        }
      }
  }
}

// ---------------------------------------------------------------------------
// pf3_kernel: pf2's tiling with a deeper pipeline (K a multiple of 64).
//
//  * Activation tiles go straight from memory to LDS (128-bit direct-to-LDS
//    buffer loads: lane l of a load lands at base + 16 l), four K steps in a
//    ring, so they need no staging registers.  LDS chunk (row, c) of 16 bytes
//    sits at position row * 8 + (c ^ ((row >> 1) & 7)): the 16 lanes that a
//    128-bit LDS read serves together (16 consecutive rows, one chunk each)
//    then cover all 64 banks (two 128-byte rows per bank line), so the
//    A-fragment reads are free of bank conflicts without padding.
//  * Weights and scales/zeros rotate through three register sets.
//  * Loads run two K steps ahead.  Every step issues the same number of
//    loads, so "this wave's activations of step t have landed" is one fixed
//    s_waitcnt vmcnt(N); a raw s_barrier then makes all waves' chunks
//    visible.  The barrier is written without a memory fence because the
//    fence would wait for every outstanding load, including the prefetched
//    ones.
//  * Software pipeline over the four 16-deep K sub-steps of a step: while
//    the MFMAs of sub-step j run, the wave reads the A fragments of j + 1
//    from LDS and dequantizes the B fragments of j + 1.  The barrier for
//    step t + 1 sits between sub-steps 2 and 3 of step t, so sub-step 3
//    already prefetches step t + 1's first fragments.  Passing that barrier
//    means every wave is done with step t - 1, whose LDS slot ((t + 3) % 4)
//    and register set ((t + 3) % 3, last dequantized during sub-step 2) are
//    then refilled for step t + 3.
// 16 bytes per lane from a raw buffer straight into LDS at lds + 16 * lane,
// the buffer offset split into a per-lane and a wave-uniform part.
__device__ __forceinline__ void lds_load16_so(__amdgpu_buffer_rsrc_t r, void* lds, uint32_t voffset,
                                              uint32_t soffset) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (__attribute__((address_space(3))) void*)lds, 16, voffset, soffset, 0, 0);
}

// KH = 2: the workgroup holds two sets of NW waves that run the same tile
// over the two halves of its K range, each with its own LDS ring, in
// lockstep (one barrier per step for all of them); the second set's
// accumulators are added to the first set's through LDS at the end, in that
// fixed order.  This puts two waves on every SIMD for tiles that would
// otherwise leave one wave per SIMD, without writing split-K partials.  The
// host uses it for 32-row tiles only: there it measured 5-7 % faster (the
// grouped q/k/v and gate/up launches at M = 128); with 64- and 128-row tiles
// the lockstep halves ran no faster than one wave per SIMD, or slower
// (down_proj at M = 2048: 71 against 68 us).
template <int DT, int NW, bool SZK, int MB, int KH, bool FIN = false>
__device__ __forceinline__ void pf3_tile(const Pf2Args& a, const int t) {
  typedef typename Act<DT>::frag F;
  static_assert(KH == 1 || KH == 2, "K halves");
  constexpr int BM = 32 * MB;        // rows per tile: MB blocks of 32
  constexpr int XL = BM / 8 / NW;    // direct-to-LDS activation loads per wave per step (1 KB each)
  static_assert(XL >= 1, "activation loads per wave");
  constexpr int NSZ = SZK ? 4 : 1;   // scale (and zero) loads per step
  constexpr int LPS = XL + 2 * NSZ + 4;  // loads per step and wave
  constexpr int WAITN = 2 * NSZ + 4 + LPS;  // loads issued after a step's activation loads
  constexpr int WAIT_IMM = (WAITN & 15) | 0x70 | 0xF00 | ((WAITN >> 4) << 14);
  constexpr int SLOT = BM * PF2_BK;  // elements of one LDS slot
  static_assert(WAITN < 64, "vmcnt range");
  __shared__ __attribute__((aligned(16))) uint16_t xs_all[KH * 4 * SLOT];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int kh = KH == 1 ? 0 : wave / NW;  // K half of this wave
  const int wn = wave - kh * NW;
  uint16_t* const xs = xs_all + kh * 4 * SLOT;
  const int l32 = lane & 31, lh = lane >> 5;
  const int split = t / a.tiles_mn;
  const int tmn = t - split * a.tiles_mn;
  const int tile_m = tmn / a.tiles_n;
  const int tile_n = tmn - tile_m * a.tiles_n;
  const int m0 = tile_m * BM;
  const int n0w = (tile_n * NW + wn) * 64;
  const int N = a.N;
  const int KT = a.K / PF2_BK;
  // KH = 2: the host gives every split the same even number of steps, so both
  // halves run the same number of steps (and barriers)
  const int kt0 = split * a.kt_per_split + kh * (a.kt_per_split / KH);
  const int nsteps = KH == 1 ? min(a.kt_per_split, KT - kt0) : a.kt_per_split / KH;

  const __amdgpu_buffer_rsrc_t rx = __builtin_amdgcn_make_buffer_rsrc((void*)a.x, (short)0, (int)a.x_bytes, 0x00020000);
  const __amdgpu_buffer_rsrc_t rq = __builtin_amdgcn_make_buffer_rsrc((void*)a.qw, (short)0, (int)a.qw_bytes, 0x00020000);
  const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc((void*)a.sc, (short)0, (int)a.sz_bytes, 0x00020000);
  const __amdgpu_buffer_rsrc_t rz = __builtin_amdgcn_make_buffer_rsrc((void*)a.ze, (short)0, (int)a.sz_bytes, 0x00020000);
  constexpr uint32_t OOB = 0x80000000u;

  // activation loads: instruction j of this wave fills LDS positions
  // [64 (wn XL + j), +64); lane l -> row 8 (wn XL + j) + l / 8, swizzled slot l % 8
  uint32_t x_off[XL];
#pragma unroll
  for (int j = 0; j < XL; ++j) {
    const int row = 8 * (wn * XL + j) + (lane >> 3);
    const int c = (lane & 7) ^ ((row >> 1) & 7);
    const int m = m0 + row;
    x_off[j] = m < a.M ? (uint32_t)((int64_t)m * a.sxm * 2) + (uint32_t)c * 16u : OOB;
  }
  // The buffer range check covers the per-lane (VGPR) offset plus the
  // immediate, not the scalar offset that carries the step: a lane whose two
  // columns lie past N (a partial last tile; N is even, so a lane's pair is
  // either inside or past the end) would read past the end of qweight (or of
  // scales / zeros) on the last k8 rows.  Those lanes take an offset the check
  // rejects, so they read zeros with no memory access; their columns are never
  // stored.  Loop invariant: the step offsets stay scalar.
  const bool col_in = n0w + 2 * l32 < N;
  const uint32_t w_lane = col_in ? ((uint32_t)lh * (uint32_t)N + (uint32_t)(n0w + 2 * l32)) * 4u : OOB;
  const uint32_t sz_col = col_in ? (uint32_t)(n0w + 2 * l32) * 2u : OOB;
  const uint32_t magic = fp16_magic_vgpr();
  // A-fragment read offsets (elements) of block mb = 0: row l32, chunk 2 ks + lh.
  // Block mb adds 32 rows (2048 elements, an immediate offset): its rows have
  // the same swizzle since (mb * 32 + l32) >> 1 & 7 == (l32 >> 1) & 7.
  int a_off[4];
#pragma unroll
  for (int ks = 0; ks < 4; ++ks) {
    const int c = ks * 2 + lh;
    a_off[ks] = (l32 * 8 + (c ^ ((l32 >> 1) & 7))) * 8;
  }

  struct Regs {
    u32x2 w[4];
    uint32_t s[NSZ], z[NSZ];
  };
  // The step enters every load through the scalar offset (the per-lane offsets
  // are loop invariant: no per-step vector address arithmetic).  Prefetches
  // past this split's last step, which no step consumes, reload that last
  // step.  With the columns past N sent out of range above, every load with
  // an in-range per-lane offset stays inside its tensor (also in a partial
  // last column tile).
  auto issue = [&](Regs& r, int st) {  // step st (0-based within this split)
    const int kt = kt0 + (st < nsteps ? st : nsteps - 1);  // scalar
    uint16_t* slot = xs + (st & 3) * SLOT;
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int j = 0; j < XL; ++j)
      lds_load16_so(rx, slot + (wn * XL + j) * 512, x_off[j], (uint32_t)kt * PF2_BK * 2u);
#pragma unroll
    for (int j = 0; j < NSZ; ++j) {
      if constexpr (SZK) {  // groups below 64: the group depends on the lane's k half
        const uint32_t g = (uint32_t)((kt * PF2_BK + j * 16 + lh * 8) >> a.gshift);
        const uint32_t off = g * (uint32_t)N * 2u + sz_col;
        r.s[j] = __builtin_amdgcn_raw_buffer_load_b32(rs, off, 0, 0);
        r.z[j] = __builtin_amdgcn_raw_buffer_load_b32(rz, off, 0, 0);
      } else {
        const uint32_t g = (uint32_t)((kt * PF2_BK) >> a.gshift);
        r.s[j] = __builtin_amdgcn_raw_buffer_load_b32(rs, sz_col, g * (uint32_t)N * 2u, 0);
        r.z[j] = __builtin_amdgcn_raw_buffer_load_b32(rz, sz_col, g * (uint32_t)N * 2u, 0);
      }
    }
    const uint32_t wso = (uint32_t)kt * 8u * (uint32_t)N * 4u;
#pragma unroll
    for (int ks = 0; ks < 4; ++ks)
      r.w[ks] = __builtin_amdgcn_raw_buffer_load_b64(rq, w_lane, wso + (uint32_t)ks * 2u * (uint32_t)N * 4u, 0);
    __builtin_amdgcn_sched_barrier(0);
  };

  f32x16 acc[MB][2];
#pragma unroll
  for (int mb = 0; mb < MB; ++mb)
#pragma unroll
    for (int nb = 0; nb < 2; ++nb)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[mb][nb][r] = 0.0f;

  // pipeline registers: A and B fragments of the sub-step being multiplied
  // and of the next one; the group constants of the step being dequantized
  F af[2][MB], bf[2][2];
  GroupConst gc[2];
  auto load_a = [&](int st, int ks, F* out) {
    const uint16_t* xb = xs + (st & 3) * SLOT;
#pragma unroll
    for (int mb = 0; mb < MB; ++mb)
      out[mb] = __builtin_bit_cast(F, *reinterpret_cast<const u32x4*>(&xb[a_off[ks] + mb * 2048]));
  };
  auto dequant_b = [&](const Regs& r, int ks, F* out) {
    if (ks == 0 || SZK) {
      const int j = SZK ? ks : 0;
#pragma unroll
      for (int nb = 0; nb < 2; ++nb)
        gc[nb] = make_group_const((uint16_t)(r.s[j] >> (16 * nb)), (uint16_t)(r.z[j] >> (16 * nb)));
    }
#pragma unroll
    for (int nb = 0; nb < 2; ++nb) out[nb] = dequant_word<DT>(r.w[ks][nb], gc[nb], magic);
  };
  auto mfma = [&](const F* af_, const F* bf_) {
#pragma unroll
    for (int mb = 0; mb < MB; ++mb)
#pragma unroll
      for (int nb = 0; nb < 2; ++nb) acc[mb][nb] = Mfma<DT>::m32(af_[mb], bf_[nb], acc[mb][nb]);
  };
  // (The order of MFMAs, LDS reads and VALU inside a sub-step is left to
  // the compiler: fixed interleave patterns of 3..12 VALU per MFMA, or MFMA
  // pairs, measured 1-6 % slower than its own schedule.)
  // wait for this wave's activation loads of the next step, then for every wave
  auto sync_step = [&]() {
    __builtin_amdgcn_sched_barrier(0);
    __builtin_amdgcn_s_waitcnt(WAIT_IMM);
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
    __builtin_amdgcn_sched_barrier(0);
  };
  // step st from register set cur; nxt holds step st + 1, and cur is
  // refilled with step st + 3 once the barrier is passed
  auto step = [&](Regs& cur, const Regs& nxt, int st) {
#pragma unroll
    for (int ks = 0; ks < 3; ++ks) {
      const int c = ks & 1;
      __builtin_amdgcn_sched_barrier(0);
      load_a(st, ks + 1, af[c ^ 1]);
      dequant_b(cur, ks + 1, bf[c ^ 1]);
      mfma(af[c], bf[c]);
      __builtin_amdgcn_sched_barrier(0);
    }
    sync_step();
    issue(cur, st + 3);
    load_a(st + 1, 0, af[0]);
    dequant_b(nxt, 0, bf[0]);
    mfma(af[1], bf[1]);
    __builtin_amdgcn_sched_barrier(0);
  };

  Regs r0, r1, r2;
  issue(r0, 0);
  issue(r1, 1);
  sync_step();
  issue(r2, 2);
  load_a(0, 0, af[0]);
  dequant_b(r0, 0, bf[0]);
  // whole register-set rotations in the loop, so that every path into its
  // head has issued the same loads in the same order (the compiler's vmcnt
  // bookkeeping then stays exact); the one or two remaining steps after it
  int st = 0;
  for (; st + 3 <= nsteps; st += 3) {
    step(r0, r1, st);
    step(r1, r2, st + 1);
    step(r2, r0, st + 2);
  }
  if (st < nsteps) step(r0, r1, st);
  if (st + 1 < nsteps) step(r1, r2, st + 1);
  __builtin_amdgcn_s_waitcnt(0);  // no load (and no LDS write) outstanding past the loop

  if constexpr (KH == 2) {
    // second half's accumulators -> LDS (lane-major, conflict-free) -> added
    // to the first half's; NW waves x MB * 2 * 16 * 64 floats fill the two rings
    constexpr int PER = MB * 2 * 16 * 64;
    static_assert(NW * PER * 4 <= KH * 4 * SLOT * 2, "partials fit the rings");
    float* const P = reinterpret_cast<float*>(xs_all) + wn * PER;
    __syncthreads();  // every wave is past its last ring read
    if (kh == 1) {
#pragma unroll
      for (int mb = 0; mb < MB; ++mb)
#pragma unroll
        for (int nb = 0; nb < 2; ++nb)
#pragma unroll
          for (int r = 0; r < 16; ++r) P[((mb * 2 + nb) * 16 + r) * 64 + lane] = acc[mb][nb][r];
    }
    __syncthreads();
    if (kh == 0) {
#pragma unroll
      for (int mb = 0; mb < MB; ++mb)
#pragma unroll
        for (int nb = 0; nb < 2; ++nb)
#pragma unroll
          for (int r = 0; r < 16; ++r) acc[mb][nb][r] += P[((mb * 2 + nb) * 16 + r) * 64 + lane];
    }
  }

  constexpr int TW = 64 * NW;  // tile width (elements)
  // FIN: K in two splits finished here (arrival counters in a.cnt): both
  // splits publish their tile (the kh == 0 waves' accumulators, lane-major
  // 16-byte chunks, as 128-bit sc1 stores: written through to the level all
  // XCDs share), wait until the stores have completed and count the
  // arrival; the second to arrive reads the other's tile with sc1 loads,
  // adds it (p0 + p1 has the same bits in either order), writes y and
  // leaves the counter at zero.  Otherwise a split writes fp32 partials for
  // the reduce launch.  (A template parameter: with the finish compiled
  // into every instantiation, the grouped launches at M = 512 / 2048
  // measured 7 us slower.)
  if constexpr (FIN) {
    constexpr int C = MB * 2 * 4;  // 16-byte accumulator chunks per lane
    constexpr uint32_t RANGE = BM * TW * sizeof(float);
    float* const parts = a.ws + (int64_t)tmn * 2 * (BM * TW);
    const __amdgpu_buffer_rsrc_t rp =
        __builtin_amdgcn_make_buffer_rsrc((void*)parts, (short)0, 2 * (int)RANGE, 0x00020000);
    const uint32_t lane_off = ((uint32_t)(wn * C) * 64u + (uint32_t)lane) * 16u;  // + 1024 c
    if (kh == 0) {
#pragma unroll
      for (int c = 0; c < C; ++c) {
        const f32x4 v = f32x4{acc[c / 8][(c / 4) % 2][4 * (c % 4)], acc[c / 8][(c / 4) % 2][4 * (c % 4) + 1],
                              acc[c / 8][(c / 4) % 2][4 * (c % 4) + 2], acc[c / 8][(c / 4) % 2][4 * (c % 4) + 3]};
        __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, v), rp,
                                               (uint32_t)split * RANGE + lane_off + 1024u * c, 0, 16);
      }
    }
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    // the arrival count goes through the ring array's last word (no second
    // LDS object: that made the compiler wait for every direct-to-LDS load in
    // flight before the main loop's fragment reads)
    unsigned* const arrived = reinterpret_cast<unsigned*>(xs_all + KH * 4 * SLOT) - 1;
    if (tid == 0) *arrived = __hip_atomic_fetch_add(a.cnt + tmn, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    __syncthreads();
    if (*arrived != 1u) return;
    if (tid == 0) __hip_atomic_store(a.cnt + tmn, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    if (kh == 0) {
      const uint32_t other = (uint32_t)(1 - split) * RANGE;
#pragma unroll
      for (int b = 0; b < 2; ++b) {  // two batches of C / 2 loads in flight
        u32x4 o[C / 2];
#pragma unroll
        for (int i = 0; i < C / 2; ++i)
          o[i] = __builtin_amdgcn_raw_buffer_load_b128(rp, other + lane_off + 1024u * (b * (C / 2) + i), 0, 16);
#pragma unroll
        for (int i = 0; i < C / 2; ++i) {
          const int c = b * (C / 2) + i;
          const f32x4 t = __builtin_bit_cast(f32x4, o[i]);
#pragma unroll
          for (int e = 0; e < 4; ++e) acc[c / 8][(c / 4) % 2][4 * (c % 4) + e] += t[e];
        }
      }
    }
  }
  // (the conditions below spelled out: a bool variable for them changed the
  // grouped launch's code, 228 -> 238 VGPRs, and made it slower)
  if (BM * TW <= 4 * SLOT && (FIN || a.ws == nullptr) && a.y16) {
    // Output through LDS: the tile (BM x 64 NW values of the output dtype,
    // when it fits the four ring slots) is assembled there, then written back
    // as 16-byte chunks, whole 64 NW-wide row segments per 64 NW / 8 lanes
    // instead of 128-byte pieces per lane pair.
    __syncthreads();  // every wave is past its last A-fragment (or partial) read
    uint32_t* T = reinterpret_cast<uint32_t*>(xs_all);
    if (kh == 0) {
#pragma unroll
      for (int mb = 0; mb < MB; ++mb)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int row = mb * 32 + 8 * (r >> 2) + 4 * lh + (r & 3);
          T[row * (TW / 2) + wn * 32 + l32] = (uint32_t)float_to_act_bits<DT>(acc[mb][0][r]) |
                                              ((uint32_t)float_to_act_bits<DT>(acc[mb][1][r]) << 16);
        }
    }
    __syncthreads();
    constexpr int CPR = TW / 8;  // 16-byte chunks per tile row
    const int n0 = tile_n * TW;
#pragma unroll 4
    for (int c = tid; c < BM * CPR; c += NW * KH * 64) {
      const int row = c / CPR, cc = c - row * CPR;
      const int m = m0 + row, n = n0 + cc * 8;
      if (m < a.M && n < N)
        // non-temporal: the output is not read again by this kernel (about
        // 2 % on the M = 2048 block against cached stores)
        __builtin_nontemporal_store(*reinterpret_cast<const u32x4*>(&T[row * (TW / 2) + cc * 4]),
                                    reinterpret_cast<u32x4*>(a.y + (int64_t)m * a.ldy + n));
    }
    return;
  }

  const int n = n0w + 2 * l32;
  if (kh == 0 && n < N) {
#pragma unroll
    for (int mb = 0; mb < MB; ++mb)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int m = m0 + mb * 32 + 8 * (r >> 2) + 4 * lh + (r & 3);
        if (m >= a.M) continue;
        if (!FIN && a.ws != nullptr) {  // fp32 partials for the reduce launch
          float2 v;
          v.x = acc[mb][0][r];
          v.y = acc[mb][1][r];
          *reinterpret_cast<float2*>(a.ws + ((int64_t)split * a.M + m) * N + n) = v;
        } else {
          const uint32_t v = (uint32_t)float_to_act_bits<DT>(acc[mb][0][r]) |
                             ((uint32_t)float_to_act_bits<DT>(acc[mb][1][r]) << 16);
          *reinterpret_cast<uint32_t*>(a.y + (int64_t)m * a.ldy + n) = v;
        }
      }
  }
}


template <int DT, int NW, bool SZK, int MB, int KH, bool FIN = false>
__global__ __launch_bounds__(NW * KH * 64) __attribute__((amdgpu_waves_per_eu(2))) void pf3_kernel(Pf2Args a) {
  pf3_tile<DT, NW, SZK, MB, KH, FIN>(a, (int)blockIdx.x);
}

// Several products sharing one activation matrix (q/k/v, gate/up) in one
// launch: problem p owns workgroups [wg_start[p], wg_start[p + 1]).
constexpr int PF3_MAX_GROUPED = 4;
struct Pf3Grouped {
  Pf2Args prob[PF3_MAX_GROUPED];
  int wg_start[PF3_MAX_GROUPED + 1];
  int count;
};

template <int DT, int NW, bool SZK, int MB, int KH>
__global__ __launch_bounds__(NW * KH * 64) __attribute__((amdgpu_waves_per_eu(2))) void pf3_grouped_kernel(Pf3Grouped g) {
  const int b = (int)blockIdx.x;
  int p = 0;
#pragma unroll
  for (int i = 1; i < PF3_MAX_GROUPED; ++i)
    if (i < g.count && b >= g.wg_start[i]) p = i;
  pf3_tile<DT, NW, SZK, MB, KH>(g.prob[p], b - g.wg_start[p]);
}

// ---------------------------------------------------------------------------
// pf5_kernel: TS x TS output tiles (TS = 64 or 128) for products with about
// one tile per CU, the weight tile dequantized ONCE per workgroup into LDS.
//
// pf3 gives every wave its own 64 columns and dequantizes them in registers
// for the wave's rows: cheap per MFMA with 128-row tiles, but a shape such as
// k_proj at M = 2048 (2048 x 512), q_proj at M = 512 (512 x 2048) or gate_proj
// at M = 128 (128 x 8192) has 256 tiles of 64 x 64 at most, so pf3 runs
// 32-row tiles whose dequantization is repeated for every 32 rows, or split-K
// with fp32 partials and a reduce launch.  Here:
//  * A set of four waves computes the tile as its 2 x 2 quarters: one
//    32 x 32 block (one v_mfma_f32_32x32x16 accumulator) per wave for
//    TS = 64, 2 x 2 such blocks per wave for TS = 128.  Per 64-k step the
//    set's 256 threads load the 8 x TS packed words (TS / 32 adjacent columns
//    of one k8 row per thread), dequantize them exactly as pf3 does (fp32
//    (q - z) * s, one rounding to the activation dtype) and store the bf16 /
//    fp16 B tile to LDS, column-major with 16-byte chunk (column n, k8 row j)
//    at slot n * 8 + (j ^ ((n >> 1) & 7)) (TS = 128: j ^ (((n >> 2) ^ (n << 1))
//    & 7), below); the activation tile arrives by
//    direct-to-LDS loads in pf3's swizzled layout, so the A and B fragment
//    reads (32 rows / columns x one chunk per 16 lanes) hit all banks.
//  * KP sets (KP = 1, 2 or 4 per workgroup, 4 to 16 waves) run the same tile
//    over KP contiguous parts of K in lockstep, each with its own LDS area
//    (2 activation slots, 2 weight buffers: 32 KB for TS = 64, 64 KB for
//    TS = 128, so KP <= 2 there); the parts are added
//    through LDS in part order at the end, so the result is a fixed function
//    of the inputs (no atomics, no partial-sum buffer, no reduce launch).
//  * One barrier per step; after it the activations of step t + 1 and the
//    packed words of step t + 2 are issued, step t is multiplied and the
//    words of step t + 1 (loaded a step earlier) are dequantized into the
//    other weight buffer.  Slots and buffers alternate with the step's
//    parity, so in the two-step loop body every LDS address is a per-lane
//    constant plus an immediate, and every load takes its step through the
//    scalar offset: the only per-step vector instructions are the
//    dequantization (52 VALU instructions per wave and step, against 74 with
//    a three-slot ring indexed at run time: 5-10 % faster on the shapes
//    below).  "The activations of step t + 1 have landed" is then
//    s_waitcnt vmcnt(3) (only the three word / scale / zero loads issued
//    after them may be outstanding).
// Measured against pf3's planned launch (bench shapes, G = 128, bf16):
// k_proj at M = 2048 17.7 -> 13.1 us (KP = 2), q_proj at M = 512 18.7 ->
// 11.7 us, k_proj at M = 512 11.5 -> 10.5 us, gate_proj at M = 128 18.9 ->
// 11.7 us (KP = 4); slower where there are more tiles than CUs (q_proj at
// M = 2048: 33.8 against 25.7 us) or K = 8192 (down_proj at M = 512: 34.8
// against 33.0 us).  TS = 128 with two K parts (eight waves, two per SIMD,
// a 64 x 64 quarter per wave) for products with 0.75 to 1 tile of 128 x 128
// per CU and K <= 4096, where pf3's plans are 64-row tiles with one wave per
// SIMD: q_proj at M = 2048 28.5 -> 26.6 us, gate_proj at M = 512 28.2 ->
// 26.2 us, 2048 x 2048 x 4096 51.3 -> 46.6 us (slower with K = 8192, with
// more tiles than CUs, or with half the CUs idle).  Sub-step software
// pipelining (pf3's fragment prefetch across the barrier) measured slower
// here.


template <int DT, int KP, int TS>
__global__ __launch_bounds__(256 * KP) void pf5_kernel(Pf2Args a) {
  typedef typename Act<DT>::frag F;
  static_assert(TS == 64 || TS == 128, "tile side");
  constexpr int WB = TS / 64;     // 32 x 32 blocks per wave side
  constexpr int XL = TS / 32;     // direct-to-LDS activation loads per thread and step
  constexpr int WPT = TS / 32;    // packed words per thread and step (adjacent columns)
  constexpr int ASLOT = TS * PF2_BK;
  constexpr int BBUF = TS * PF2_BK;
  constexpr int SET = 4 * TS * PF2_BK;  // one K part: two activation slots, two weight buffers
  // at the barrier of step t + 1 only the word / scale / zero loads of step
  // t + 2 (issued after the activations of step t + 1) may be outstanding
  constexpr int WAIT3 = 3 | 0x70;  // vmcnt(3), lgkmcnt(0)
  constexpr int WAIT0 = 0 | 0x70;  // vmcnt(0), lgkmcnt(0)
  __shared__ __attribute__((aligned(16))) uint16_t lds[KP * SET];
  constexpr uint32_t OOB = 0x80000000u;

  const int lane = threadIdx.x & 63;
  const int kp = KP == 1 ? 0 : __builtin_amdgcn_readfirstlane((int)threadIdx.x >> 8);  // K part
  const int tid = threadIdx.x & 255;                                                  // within the part
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  uint16_t* const As = lds + kp * SET;
  uint16_t* const Bs = As + 2 * ASLOT;
  const int wm = wave >> 1, wn = wave & 1;  // this wave's quarter of the tile
  const int l32 = lane & 31, lh = lane >> 5;
  static_assert(TS == 64 || KP == 2, "128-wide tiles run two K parts");
  const int KS = a.ks;  // K ranges across workgroups
  const int split = KS > 1 ? (int)blockIdx.x / a.tiles_mn : 0;
  const int tb = (int)blockIdx.x - split * a.tiles_mn;  // the tile
  const int tile_m = tb / a.tiles_n;
  const int tile_n = tb - tile_m * a.tiles_n;
  const int m0 = tile_m * TS, n0 = tile_n * TS;
  const int N = a.N;
  const int KT = a.kt_per_split;  // steps of one part (even, >= 2; the host divides K)
  const int kt0 = (split * KP + kp) * KT;

  const __amdgpu_buffer_rsrc_t rx = __builtin_amdgcn_make_buffer_rsrc((void*)a.x, (short)0, (int)a.x_bytes, 0x00020000);
  const __amdgpu_buffer_rsrc_t rq = __builtin_amdgcn_make_buffer_rsrc((void*)a.qw, (short)0, (int)a.qw_bytes, 0x00020000);
  const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc((void*)a.sc, (short)0, (int)a.sz_bytes, 0x00020000);
  const __amdgpu_buffer_rsrc_t rz = __builtin_amdgcn_make_buffer_rsrc((void*)a.ze, (short)0, (int)a.sz_bytes, 0x00020000);

  // per-lane offsets are loop invariant; the step enters through the scalar
  // offset of each load (no per-step address arithmetic in the vector ALU)
  uint32_t x_off[XL];
#pragma unroll
  for (int i = 0; i < XL; ++i) {
    const int row = 8 * (wave * XL + i) + (lane >> 3);
    const int c = (lane & 7) ^ ((row >> 1) & 7);
    const int m = m0 + row;
    x_off[i] = m < a.M ? (uint32_t)((int64_t)m * a.sxm * 2) + (uint32_t)c * 16u : OOB;
  }
  const int wj = tid >> 5;          // k8 row of this thread's words
  const int wc = WPT * (tid & 31);  // first of its WPT adjacent columns
  const uint32_t w_off = ((uint32_t)wj * (uint32_t)N + (uint32_t)(n0 + wc)) * 4u;
  const uint32_t sz_off = (uint32_t)(n0 + wc) * 2u;
  // weight chunk (column n, k8 row j) of a buffer at slot n * 8 + (j ^ bswz(n)),
  // elements.  A 128-bit LDS write serves 8 lanes at a time, a 128-bit read 16
  // lanes over the 64 banks (even and odd columns in the two bank halves).
  // TS = 64: the 8 lanes of a store hold columns 2l + i, and (n >> 1) & 7
  // gives them 8 distinct chunks, as it gives the 8 even (odd) columns of a
  // fragment read.  TS = 128: a store's 8 lanes hold columns 4l + i, where
  // (n >> 1) & 7 takes only 4 values (a two-way conflict on every store);
  // ((n >> 2) ^ (n << 1)) & 7 is distinct over both sets.  Both depend on
  // n % 32 only, so blocks 32 columns apart share the offsets.
  auto bswz = [](int n) { return TS == 64 ? ((n >> 1) & 7) : (((n >> 2) ^ (n << 1)) & 7); };
  int b_off[WPT];
#pragma unroll
  for (int i = 0; i < WPT; ++i) b_off[i] = ((wc + i) * 8 + (wj ^ bswz(wc + i))) * 8;
  const uint32_t magic = fp16_magic_vgpr();

  struct Regs {
    uint32_t w[WPT];
    uint32_t s[WPT / 2], z[WPT / 2];
  };
  auto issue_w = [&](Regs& r, int st) {
    const int t = kt0 + st;
    const uint32_t g = (uint32_t)((t * PF2_BK) >> a.gshift);
    const uint32_t wso = (uint32_t)t * 8u * (uint32_t)N * 4u, sso = g * (uint32_t)N * 2u;
    if constexpr (WPT == 4) {
      const u32x4 w = __builtin_amdgcn_raw_buffer_load_b128(rq, w_off, wso, 0);
      const u32x2 s = __builtin_amdgcn_raw_buffer_load_b64(rs, sz_off, sso, 0);
      const u32x2 z = __builtin_amdgcn_raw_buffer_load_b64(rz, sz_off, sso, 0);
#pragma unroll
      for (int i = 0; i < 4; ++i) r.w[i] = w[i];
#pragma unroll
      for (int i = 0; i < 2; ++i) {
        r.s[i] = s[i];
        r.z[i] = z[i];
      }
    } else {
      const u32x2 w = __builtin_amdgcn_raw_buffer_load_b64(rq, w_off, wso, 0);
      r.w[0] = w[0];
      r.w[1] = w[1];
      r.s[0] = __builtin_amdgcn_raw_buffer_load_b32(rs, sz_off, sso, 0);
      r.z[0] = __builtin_amdgcn_raw_buffer_load_b32(rz, sz_off, sso, 0);
    }
  };
  auto issue_a = [&](int st, int slot) {
    const int t = kt0 + st;
    uint16_t* base = As + slot * ASLOT;
#pragma unroll
    for (int i = 0; i < XL; ++i)
      lds_load16_so(rx, base + (wave * XL + i) * 512, x_off[i], (uint32_t)t * 128u);
  };
  auto dequant = [&](const Regs& r, int b) {
    uint16_t* buf = Bs + b * BBUF;
#pragma unroll
    for (int i = 0; i < WPT; ++i) {
      const GroupConst gc = make_group_const((uint16_t)(r.s[i >> 1] >> (16 * (i & 1))), (uint16_t)(r.z[i >> 1] >> (16 * (i & 1))));
      const F f = dequant_word<DT>(r.w[i], gc, magic);
      *reinterpret_cast<u32x4*>(buf + b_off[i]) = __builtin_bit_cast(u32x4, f);
    }
  };

  f32x16 acc[WB][WB];
#pragma unroll
  for (int i = 0; i < WB; ++i)
#pragma unroll
    for (int j = 0; j < WB; ++j)
#pragma unroll
      for (int e = 0; e < 16; ++e) acc[i][j][e] = 0.0f;
  int f_off[4], fb_off[4];
#pragma unroll
  for (int ks = 0; ks < 4; ++ks) {
    f_off[ks] = (l32 * 8 + ((2 * ks + lh) ^ ((l32 >> 1) & 7))) * 8;
    fb_off[ks] = TS == 64 ? f_off[ks] : (l32 * 8 + ((2 * ks + lh) ^ bswz(l32))) * 8;
  }
  // blocks 32 rows / columns apart have the same swizzle: an immediate offset
  auto multiply = [&](int slot) {
    const uint16_t* A = As + slot * ASLOT + wm * (TS / 2) * PF2_BK;
    const uint16_t* B = Bs + slot * BBUF + wn * (TS / 2) * PF2_BK;
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) {
      F af[WB], bf[WB];
#pragma unroll
      for (int i = 0; i < WB; ++i) {
        af[i] = __builtin_bit_cast(F, *reinterpret_cast<const u32x4*>(A + i * 32 * PF2_BK + f_off[ks]));
        bf[i] = __builtin_bit_cast(F, *reinterpret_cast<const u32x4*>(B + i * 32 * PF2_BK + fb_off[ks]));
      }
#pragma unroll
      for (int i = 0; i < WB; ++i)
#pragma unroll
        for (int j = 0; j < WB; ++j) acc[i][j] = Mfma<DT>::m32(af[i], bf[j], acc[i][j]);
    }
  };
  auto sync3 = [&]() {
    __builtin_amdgcn_sched_barrier(0);
    __builtin_amdgcn_s_waitcnt(WAIT3);
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
    __builtin_amdgcn_sched_barrier(0);
  };
  auto sync0 = [&]() {
    __builtin_amdgcn_sched_barrier(0);
    __builtin_amdgcn_s_waitcnt(WAIT0);
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
    __builtin_amdgcn_sched_barrier(0);
  };

  // step t: activations of t + 1 and words of t + 2 issued, step t
  // multiplied (slot and buffer t & 1), words of t + 1 dequantized into
  // buffer (t + 1) & 1; register set t & 1 receives the words of t + 2
  Regs r0, r1;
  issue_a(0, 0);
  issue_w(r0, 0);
  issue_w(r1, 1);
  dequant(r0, 0);
  int st = 0;
  for (; st + 2 < KT; st += 2) {
    sync3();
    __builtin_amdgcn_sched_barrier(0);
    issue_a(st + 1, 1);
    issue_w(r0, st + 2);
    __builtin_amdgcn_sched_barrier(0);
    multiply(0);
    dequant(r1, 1);
    sync3();
    __builtin_amdgcn_sched_barrier(0);
    issue_a(st + 2, 0);
    issue_w(r1, st + 3);
    __builtin_amdgcn_sched_barrier(0);
    multiply(1);
    dequant(r0, 0);
  }
  // the last two steps: no words left to load
  sync3();
  issue_a(st + 1, 1);
  __builtin_amdgcn_sched_barrier(0);
  multiply(0);
  dequant(r1, 1);
  sync0();
  multiply(1);
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();

  constexpr int PER = WB * WB * 16;  // accumulator floats per lane
  // 128-wide tiles with K cut across workgroups: part p keeps block row
  // i == p of its wave's 2 x 2 blocks (`own`), so that all eight waves share
  // the publishing and the last range's reads
  const bool scattered = TS == 128 && KS > 1;
  f32x16 own[WB];
  if constexpr (TS == 128) {
    if (scattered) {
      // each part hands the other its other block row through LDS; the sum
      // p0 + p1 has the same bits in either part (IEEE addition commutes)
      float* const X = reinterpret_cast<float*>(lds);
      float* const Xw = X + (kp * 4 + wave) * (WB * 16) * 64 + lane;
#pragma unroll
      for (int j = 0; j < WB; ++j)
#pragma unroll
        for (int e = 0; e < 16; ++e) Xw[(j * 16 + e) * 64] = kp == 0 ? acc[1][j][e] : acc[0][j][e];
      __syncthreads();
      const float* const Xr = X + ((1 - kp) * 4 + wave) * (WB * 16) * 64 + lane;
#pragma unroll
      for (int j = 0; j < WB; ++j)
#pragma unroll
        for (int e = 0; e < 16; ++e) own[j][e] = (kp == 0 ? acc[0][j][e] : acc[1][j][e]) + Xr[(j * 16 + e) * 64];
    }
  }
  if (KP > 1 && !scattered) {
    // parts 1..KP-1 -> LDS (lane-major, conflict-free) -> added to part 0 in part
    // order.  Part p's wave w writes its accumulators at P + (p * 4 + w) * PER *
    // 64, element e of the lane at e * 64 + lane (slot 0 unused: every store
    // offset is a non-negative immediate, so the stores pair up)
    static_assert(KP * 4 * PER * 64 * 4 <= KP * SET * 2, "partials fit the parts' areas");
    float* const P = reinterpret_cast<float*>(lds) + wave * PER * 64 + lane;
    if (kp > 0) {
      float* const Pw = P + kp * 4 * PER * 64;
#pragma unroll
      for (int i = 0; i < WB; ++i)
#pragma unroll
        for (int j = 0; j < WB; ++j)
#pragma unroll
          for (int e = 0; e < 16; ++e) Pw[((i * WB + j) * 16 + e) * 64] = acc[i][j][e];
    }
    __syncthreads();
    if (kp == 0) {
#pragma unroll
      for (int p = 1; p < KP; ++p)
#pragma unroll
        for (int i = 0; i < WB; ++i)
#pragma unroll
          for (int j = 0; j < WB; ++j)
#pragma unroll
            for (int e = 0; e < 16; ++e) acc[i][j][e] += P[(p * 4 * PER + (i * WB + j) * 16 + e) * 64];
    }
    __syncthreads();
  }
  if (KS > 1) {
    // K split across workgroups: the publishing waves (part 0's for 64-wide
    // tiles, all eight for 128-wide ones) store the workgroup's sum (their
    // accumulators, lane-major 16-byte chunks) with 128-bit sc1 stores (the
    // cache policy of agent-scope atomic stores: written through to the
    // level all XCDs share), wait until they have completed, and count the
    // arrival; the last range to arrive reads the others with sc1 loads,
    // sums all ranges in range order (so the result does not depend on which
    // is last), leaves the counter at zero and writes the tile.
    constexpr int C = TS == 64 ? PER / 4 : WB * 4;  // 16-byte chunks per publishing lane
    const bool pub = TS == 128 || kp == 0;
    const int pw = TS == 128 ? kp * 4 + wave : wave;  // publishing wave
    f32x4 mine[C];
#pragma unroll
    for (int c = 0; c < C; ++c)
#pragma unroll
      for (int e = 0; e < 4; ++e) mine[c][e] = TS == 64 ? acc[0][0][4 * c + e] : own[(c / 4) % WB][4 * (c % 4) + e];
    float* const parts = a.ws + (int64_t)tb * KS * (TS * TS);
    const __amdgpu_buffer_rsrc_t rp = __builtin_amdgcn_make_buffer_rsrc((void*)parts, (short)0,
                                                                         KS * TS * TS * (int)sizeof(float), 0x00020000);
    const uint32_t lane_off = ((uint32_t)(pw * C) * 64u + (uint32_t)lane) * 16u;  // + 1024 c
    constexpr uint32_t RANGE = TS * TS * sizeof(float);
    if (pub) {
#pragma unroll
      for (int c = 0; c < C; ++c)
        __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, mine[c]), rp,
                                               (uint32_t)split * RANGE + lane_off + 1024u * c, 0, 16);
    }
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    // the arrival count goes through the array's last word, which neither
    // the part sums (its first half) nor, from here on, the rings use (a
    // second LDS object made the compiler wait for every direct-to-LDS load
    // in flight before each fragment read of the main loop)
    unsigned* const arrived = reinterpret_cast<unsigned*>(lds + KP * SET) - 1;
    if (threadIdx.x == 0)
      *arrived = __hip_atomic_fetch_add(a.cnt + tb, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    __syncthreads();
    if (*arrived != (unsigned)(KS - 1)) return;
    if (threadIdx.x == 0) __hip_atomic_store(a.cnt + tb, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    if (pub) {
      // every other range's chunks are requested before the first add:
      // slot o holds range o + (o >= split), so the registers are indexed
      // at compile time
      u32x4 other[kMaxPf5Split - 1][C];
#pragma unroll
      for (int o = 0; o < kMaxPf5Split - 1; ++o)
        if (o < KS - 1) {
          const uint32_t q = (uint32_t)(o + (o >= split ? 1 : 0));
#pragma unroll
          for (int c = 0; c < C; ++c)
            other[o][c] = __builtin_amdgcn_raw_buffer_load_b128(rp, q * RANGE + lane_off + 1024u * c, 0, 16);
        }
#pragma unroll
      for (int c = 0; c < C; ++c) {
        f32x4 sum = mine[c];
#pragma unroll
        for (int q = 0; q < kMaxPf5Split; ++q) {
          if (q < KS) {
            // range q in range order: slot q below this workgroup's range,
            // slot q - 1 above it (the whole vector is bit-cast: a bit cast
            // of one element of an ext_vector_type value reads the vector's
            // first element)
            const f32x4 below = __builtin_bit_cast(f32x4, other[q < kMaxPf5Split - 1 ? q : 0][c]);
            const f32x4 above = __builtin_bit_cast(f32x4, other[q > 0 ? q - 1 : 0][c]);
            const f32x4 t = q < split ? below : q == split ? mine[c] : above;
            sum = q == 0 ? t : sum + t;
          }
        }
        mine[c] = sum;
      }
#pragma unroll
      for (int c = 0; c < C; ++c)
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          if constexpr (TS == 64)
            acc[0][0][4 * c + e] = mine[c][e];
          else
            own[(c / 4) % WB][4 * (c % 4) + e] = mine[c][e];
        }
    }
  }
  // output: the tile in LDS (part 0's area), then 16-byte row chunks
  static_assert(TS * TS <= SET, "output tile fits part 0's area");
  uint16_t* T = lds;
  if (scattered) {
    // part p holds block row p of its wave's quarter
#pragma unroll
    for (int j = 0; j < WB; ++j)
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        const int row = wm * (TS / 2) + kp * 32 + 8 * (e >> 2) + 4 * lh + (e & 3);
        T[row * TS + wn * (TS / 2) + j * 32 + l32] = float_to_act_bits<DT>(own[j][e]);
      }
  } else if (kp == 0) {
#pragma unroll
    for (int i = 0; i < WB; ++i)
#pragma unroll
      for (int j = 0; j < WB; ++j)
#pragma unroll
        for (int e = 0; e < 16; ++e) {
          const int row = wm * (TS / 2) + i * 32 + 8 * (e >> 2) + 4 * lh + (e & 3);
          T[row * TS + wn * (TS / 2) + j * 32 + l32] = float_to_act_bits<DT>(acc[i][j][e]);
        }
  }
  __syncthreads();
  constexpr int CPR = TS / 8;  // 16-byte chunks per tile row
  if (a.y16) {
    for (int c = threadIdx.x; c < TS * CPR; c += 256 * KP) {
      const int row = c / CPR, cc = c - row * CPR;
      const int m = m0 + row;
      if (m < a.M)
        __builtin_nontemporal_store(*reinterpret_cast<const u32x4*>(&T[row * TS + cc * 8]),
                                    reinterpret_cast<u32x4*>(a.y + (int64_t)m * a.ldy + n0 + cc * 8));
    }
  } else {
    for (int c = threadIdx.x; c < TS * TS; c += 256 * KP) {
      const int row = c / TS, col = c - row * TS;
      const int m = m0 + row;
      if (m < a.M) a.y[(int64_t)m * a.ldy + n0 + col] = T[c];
    }
  }
}
}  // namespace w4

using namespace w4host;

namespace {

struct Pf2Plan {
  int nw = 0, mb = 4, kh = 1, splits = 1, kt_per_split = 0, tiles_n = 0, tiles_mn = 0;
  bool fin = false;  // two K splits finished in the kernel (no reduce launch)
  size_t ws = 0;
};

// Static launch table (pure function of the shape and the CU count).  Cost
// model, fitted to MI355X timings of pf3 on the Llama shapes (M = 32..2048):
// a wave alone on its SIMD needs STEP[mb] per K step of 64 (1.07 / 0.74 /
// 0.49 us for 128 / 64 / 32-row tiles); SIMDs holding k > 1 waves run them
// at 0.9 k STEP; four-wave workgroups on fewer workgroups than CUs lose 7 %
// (two-wave ones spread over more CUs); every launch costs about 3 us of
// prologue and epilogue latency plus its output bytes at 5 TB/s; split-K
// writes fp32 partials instead and adds the reduce kernel (2.2 us plus the
// partials read at 8 TB/s).
// Best plan with at most max_splits K splits; *t_est (if given) receives the
// model's time for it, in seconds.
Pf2Plan plan_pf2(int64_t M, int64_t N, int64_t K, int max_splits = 8, double* t_est = nullptr) {
  const int cus = device_cu_count();
  const int64_t KT = (K + w4::PF2_BK - 1) / w4::PF2_BK;
  Pf2Plan best;
  double best_t = 1e30;
  for (int mb : {4, 2, 1}) {
    if (mb != 4 && K % w4::PF2_BK != 0) continue;  // the register-staged kernel has 128-row tiles only
    const double step = mb == 4 ? 1.07e-6 : mb == 2 ? 0.74e-6 : 0.49e-6;
    const int64_t bm = 32 * mb;
    const int64_t tm = (M + bm - 1) / bm;
    for (int nw : {4, 2}) {
      const int64_t tn = (N + 64 * nw - 1) / (64 * nw);
      for (int s : {1, 2, 4, 8}) {
        if (s > max_splits) continue;
        const int64_t T = (KT + s - 1) / s;
        const int64_t S = (KT + T - 1) / T;
        if (S != s || (s > 1 && T < 4)) continue;
        for (int kh : {1, 2}) {
        // two K halves per workgroup: 32-row tiles and four-wave sets only,
        // every split the same even number of steps (both halves run in
        // lockstep)
        if (kh == 2 && (mb != 1 || nw != 4 || K % w4::PF2_BK != 0 || T % 2 != 0 || S * T != KT || T < 8))
          continue;
        const int64_t wgs = tm * tn * S;
        // waves per SIMD on the busiest CU: a fractional round (e.g. 1.5
        // workgroups per CU) costs the CUs that hold two as much as a full one
        const double per_simd = (double)((wgs + cus - 1) / cus * nw * kh) / 4.0;
        double t = (double)(T / kh) * step * (per_simd <= 1.0 ? 1.0 : 0.9 * per_simd);
        if (nw == 2) t *= 1.3;  // 128-column tiles: each activation tile feeds half the MFMAs
        if (nw == 4 && wgs < cus) t *= 1.07;
        if (kh == 2) t += 0.7e-6;  // the halves' sum through LDS
        t += 3e-6;
        if (S > 1) {
          const double part = (double)S * M * N * 4;
          t += part / 5e12 + 3.0e-6 + part / 8e12;  // partials written, reduce launch, read back
        } else {
          t += (double)M * N * 2 / 5e12;
        }
        if (t < best_t * 0.97) {
          best_t = t;
          best.nw = nw;
          best.mb = mb;
          best.kh = kh;
          best.splits = (int)S;
          best.kt_per_split = (int)T;
          best.tiles_n = (int)tn;
          best.tiles_mn = (int)(tm * tn);
          best.ws = S > 1 ? (size_t)S * M * N * sizeof(float) : 0;
        }
        }
      }
    }
  }
  if (t_est != nullptr) *t_est = best_t;
  // two K splits of the register-staged kernel on 128 x 256 tiles (down_proj
  // at M = 2048): the second to finish adds the first's tile (partials
  // [tile][2][128 x 256]; one arrival counter per tile), no reduce launch
  if (best.splits == 2 && best.nw == 4 && best.mb == 4 && best.kh == 1 && K % w4::PF2_BK == 0 &&
      (size_t)best.tiles_mn * 4 <= W4_WORKSPACE_COUNTER_BYTES) {
    best.fin = true;
    best.ws = (size_t)best.tiles_mn * 2 * (32 * best.mb) * (64 * best.nw) * sizeof(float);
  }
  return best;
}

bool pf2_ok(const void* x, int64_t M, int64_t N, int64_t K, int64_t sxm, int64_t sxk, const void* qw,
            const void* sc, const void* ze, const void* y, int64_t ldy) {
  return sxk == 1 && (uintptr_t)x % 16 == 0 && sxm % 8 == 0 && N % 2 == 0 && (uintptr_t)qw % 8 == 0 &&
         (uintptr_t)sc % 4 == 0 && (uintptr_t)ze % 4 == 0 && (uintptr_t)y % 4 == 0 && ldy % 2 == 0 &&
         M < (1LL << 30) && ((M - 1) * sxm + K) * 2 < (1LL << 31) && (K / 8) * N * 4 < (1LL << 31);
}

template <int DT, int NW, int MB, int KH>
void pf3_launch_k(const Pf2Plan& p, bool szk, const w4::Pf2Args& a, hipStream_t st) {
  const dim3 grid((unsigned)(p.tiles_mn * p.splits)), block(NW * KH * 64);
  if constexpr (NW == 4 && MB == 4 && KH == 1) {
    if (p.fin) {  // (the plan sets fin for this tiling only)
      if (szk)
        hipLaunchKernelGGL((w4::pf3_kernel<DT, NW, true, MB, KH, true>), grid, block, 0, st, a);
      else
        hipLaunchKernelGGL((w4::pf3_kernel<DT, NW, false, MB, KH, true>), grid, block, 0, st, a);
      return;
    }
  }
  if (szk)
    hipLaunchKernelGGL((w4::pf3_kernel<DT, NW, true, MB, KH>), grid, block, 0, st, a);
  else
    hipLaunchKernelGGL((w4::pf3_kernel<DT, NW, false, MB, KH>), grid, block, 0, st, a);
}

template <int DT, int NW, int MB>
void pf3_launch_g(const Pf2Plan& p, bool szk, const w4::Pf2Args& a, hipStream_t st) {
  if constexpr (NW == 4 && MB == 1) {
    if (p.kh == 2) {
      pf3_launch_k<DT, NW, MB, 2>(p, szk, a, st);
      return;
    }
  }
  pf3_launch_k<DT, NW, MB, 1>(p, szk, a, st);
}

template <int DT, int NW>
void pf2_launch_g(const Pf2Plan& p, bool szk, const w4::Pf2Args& a, hipStream_t st) {
  const dim3 grid((unsigned)(p.tiles_mn * p.splits)), block(NW * 64);
  if (a.K % w4::PF2_BK == 0) {  // deep pipeline: whole K steps only
    if (p.mb == 4)
      pf3_launch_g<DT, NW, 4>(p, szk, a, st);
    else if (p.mb == 2)
      pf3_launch_g<DT, NW, 2>(p, szk, a, st);
    else
      pf3_launch_g<DT, NW, 1>(p, szk, a, st);
  } else if (szk) {
    hipLaunchKernelGGL((w4::pf2_kernel<DT, NW, true>), grid, block, 0, st, a);
  } else {
    hipLaunchKernelGGL((w4::pf2_kernel<DT, NW, false>), grid, block, 0, st, a);
  }
}

// pf5 (TS x TS tiles, the weight tile dequantized once per workgroup into
// LDS) for dense rows with group sizes >= 64 (one group per 64-k step), a
// multiple of 128 per K part; K <= 4096 unless K is also cut across
// workgroups (the last two cases).  parts = K parts per workgroup (0: not
// this kernel).
//  * TS = 64 where the product has at most one 64 x 64 tile per CU (N % 64
//    == 0): four parts except for tall products (M > N), which measured
//    faster with two (k_proj at M = 2048: 13.1 against 14.3 us; q_proj at
//    M = 512 11.7 against 12.4 us, gate_proj at M = 128 11.7 against 12.3 us
//    with four).
//  * TS = 128 with two parts where it has 0.75 to 1 tile of 128 x 128 per CU
//    (N % 128 == 0, K % 256 == 0).
//  * K > 4096 with 64 < M <= 128 (down_proj at M = 128): 64 x 64 tiles of
//    four parts, K cut into ks ranges of at most 2048 over as many
//    workgroups while the launch fits one workgroup per CU, finished by the
//    last range to arrive: down_proj at M = 128 15.1 us against 17.1 us as
//    16-row slices (the decode regime's route for these rows otherwise).
//    Products of more than 128 rows with at most half a 64 x 64 tile per CU
//    (k/v at M = 512) take the same split.
//  * K > 4096 with more than 128 rows and fewer 128 x 128 tiles than CUs
//    (down_proj at M = 512 / 1024): 128 x 128 tiles of two parts, K cut into
//    ks = 2 or 4 ranges of at most 4096 while the launch fills 3/4 to all of
//    the CUs, each part keeping half of the tile's sum so that all eight
//    waves share the last range's reads.  Against pf3 (split-K and the
//    reduce launch): M x N x K = 512 x 2048 x 8192 30.9 vs 34.8 us, 1024 x
//    2048 x 8192 47.6 vs 50.1, 256 x 4096 x 8192 30.8 vs 34.5, 384 x 2048 x
//    8192 28.9 vs 31.1; ranges of 7168 (512 x 4096 x 14336) 79.1 vs 72.6.
struct Pf5Plan {
  int parts = 0, ts = 64, ks = 1;
};
Pf5Plan pf5_plan(int64_t M, int64_t N, int64_t K, int64_t G) {
  Pf5Plan p;
  const int64_t cus = device_cu_count();
  if (K > 4096 && M > 128) {
    const int64_t t128 = (M + 127) / 128 * (N / 128);
    if (G < 64 || N % 128 != 0) return p;
    int ks = 2;
    while (2 * ks <= w4::kMaxPf5Split && t128 * ks * 2 <= cus) ks *= 2;
    if (t128 * ks <= cus && 4 * t128 * ks >= 3 * cus && K % (256 * ks) == 0 && K / ks <= 4096) {
      p.parts = 2;
      p.ts = 128;
      p.ks = ks;
    }
    return p;
  }
  if (K > 4096) {
    if (G < 64 || M <= 64 || N % 64 != 0) return p;
    int ks = 2;
    while (K / ks > 2048) ks *= 2;
    if (ks <= w4::kMaxPf5Split && K % ks == 0 && (K / ks) % 512 == 0 && (M + 63) / 64 * (N / 64) * ks <= cus) {
      p.parts = 4;
      p.ks = ks;
    }
    return p;
  }
  if (G < 64 || K % 128 != 0) return p;
  if (M > 128 && N % 64 == 0 && K % 2048 == 0 && (M + 63) / 64 * (N / 64) * 2 <= cus) {
    // at most half a workgroup per CU (k/v at M = 512: 64 tiles): the same
    // K split, the ranges doubled while they fill more CUs (k/v at M = 512
    // 10.5 -> 9.5 us with four)
    int ks = 1;
    while (2 * ks <= w4::kMaxPf5Split && (M + 63) / 64 * (N / 64) * ks * 2 <= cus && (K / (ks * 2)) % 512 == 0)
      ks *= 2;
    p.parts = 4;
    p.ks = ks;
    return p;
  }
  if (N % 64 == 0 && (M + 63) / 64 * (N / 64) <= cus) {
    p.parts = (K % 512 == 0 && M <= N) ? 4 : K % 256 == 0 ? 2 : 1;
    return p;
  }
  const int64_t t128 = (M + 127) / 128 * (N / 128);
  if (N % 128 == 0 && K % 256 == 0 && 4 * t128 >= 3 * cus && t128 <= cus) {
    p.parts = 2;
    p.ts = 128;
  }
  return p;
}

// Partial-tile bytes of a K-split pf5 launch (0 when the shape takes none);
// the plan does not depend on the group size once it is >= 64.
size_t pf5_split_scratch(int64_t M, int64_t N, int64_t K) {
  const Pf5Plan p = pf5_plan(M, N, K, 64);
  return p.ks > 1 ? (size_t)p.ks * ((M + p.ts - 1) / p.ts) * (N / p.ts) * p.ts * p.ts * sizeof(float) : 0;
}

template <int DT>
void pf5_launch(const Pf5Plan& p, const w4::Pf2Args& a, hipStream_t st) {
  const dim3 grid((unsigned)(((a.M + p.ts - 1) / p.ts) * (a.N / p.ts) * p.ks));
  if (p.ts == 128)
    hipLaunchKernelGGL((w4::pf5_kernel<DT, 2, 128>), grid, dim3(512), 0, st, a);
  else if (p.parts == 4)
    hipLaunchKernelGGL((w4::pf5_kernel<DT, 4, 64>), grid, dim3(1024), 0, st, a);
  else if (p.parts == 2)
    hipLaunchKernelGGL((w4::pf5_kernel<DT, 2, 64>), grid, dim3(512), 0, st, a);
  else
    hipLaunchKernelGGL((w4::pf5_kernel<DT, 1, 64>), grid, dim3(256), 0, st, a);
}

}  // namespace

int w4_splitk_reduce_launch(const float* ws, int S, int64_t M, int64_t N, int x_dtype, void* y, int64_t ldy,
                            hipStream_t st);

// Scratch bytes (past the workspace's counter area) of a prefill launch.
size_t w4_prefill_workspace_bytes(int64_t M, int64_t N, int64_t K) {
  return std::max(plan_pf2(M, N, K).ws, pf5_split_scratch(M, N, K));
}

// True when w4_prefill_launch takes the K-split pf5 launch for this product
// (the GEMM entry point then routes such rows here instead of to the decode
// kernel's row slices).
bool w4_prefill_split_route(const void* x, int64_t M, int64_t N, int64_t K, int64_t sxm, int64_t sxk,
                            const int32_t* qw, const uint16_t* sc, const uint16_t* ze, int G, const void* y,
                            int64_t ldy) {
  return pf2_ok(x, M, N, K, sxm, sxk, qw, sc, ze, y, ldy) && pf5_plan(M, N, K, G).ks > 1;
}

int w4_prefill_launch(const void* x, int x_dtype, int64_t M, int64_t N, int64_t K, int64_t sxm,
                      int64_t sxk, const int32_t* qw, const uint16_t* sc, const uint16_t* ze, int G,
                      void* y, int64_t ldy, void* ws, size_t ws_bytes, unsigned* counters, hipStream_t st);

// The pipelined MFMA kernel for 17 <= M <= 64 as well: returns
// W4_ERR_UNSUPPORTED (nothing launched, no message) when the activations are
// not dense 16-byte-aligned rows or K is not a multiple of 64; the caller then
// takes the split-K skinny kernel.
int w4_prefill_fast_launch(const void* x, int x_dtype, int64_t M, int64_t N, int64_t K, int64_t sxm,
                           int64_t sxk, const int32_t* qw, const uint16_t* sc, const uint16_t* ze, int G,
                           void* y, int64_t ldy, void* ws, size_t ws_bytes, unsigned* counters, hipStream_t st) {
  if (K % w4::PF2_BK != 0 || !pf2_ok(x, M, N, K, sxm, sxk, qw, sc, ze, y, ldy)) return W4_ERR_UNSUPPORTED;
  return w4_prefill_launch(x, x_dtype, M, N, K, sxm, sxk, qw, sc, ze, G, y, ldy, ws, ws_bytes, counters, st);
}

int w4_prefill_launch(const void* x, int x_dtype, int64_t M, int64_t N, int64_t K, int64_t sxm,
                      int64_t sxk, const int32_t* qw, const uint16_t* sc, const uint16_t* ze, int G,
                      void* y, int64_t ldy, void* ws, size_t ws_bytes, unsigned* counters, hipStream_t st) {
  if (pf2_ok(x, M, N, K, sxm, sxk, qw, sc, ze, y, ldy)) {
    if (const Pf5Plan p5 = pf5_plan(M, N, K, G); p5.parts) {
      const int64_t tiles = ((M + p5.ts - 1) / p5.ts) * (N / p5.ts);
      if (p5.ks > 1) {
        const size_t need = (size_t)p5.ks * tiles * p5.ts * p5.ts * sizeof(float);
        if (counters == nullptr || ws == nullptr || ws_bytes < need)
          return fail(W4_ERR_WORKSPACE, "w4a16_gemm: workspace of %zu bytes required, %zu given",
                      (size_t)W4_WORKSPACE_COUNTER_BYTES + need, ws ? ws_bytes : (size_t)0);
      }
      w4::Pf2Args a{};
      a.ks = p5.ks;
      a.tiles_mn = (int)tiles;
      a.kt_per_split = (int)(K / w4::PF2_BK / p5.parts / p5.ks);
      a.ws = p5.ks > 1 ? static_cast<float*>(ws) : nullptr;
      a.cnt = p5.ks > 1 ? counters : nullptr;
      a.x = static_cast<const uint16_t*>(x);
      a.qw = reinterpret_cast<const uint32_t*>(qw);
      a.sc = sc;
      a.ze = ze;
      a.y = static_cast<uint16_t*>(y);
      a.sxm = sxm;
      a.ldy = ldy;
      a.x_bytes = (uint32_t)(((M - 1) * sxm + K) * 2);
      a.qw_bytes = (uint32_t)((K / 8) * N * 4);
      a.sz_bytes = (uint32_t)((K / G) * N * 2);
      a.M = (int)M;
      a.N = (int)N;
      a.K = (int)K;
      a.gshift = ilog2(G);
      a.tiles_n = (int)(N / p5.ts);
      a.y16 = (ldy % 8 == 0 && (uintptr_t)y % 16 == 0) ? 1 : 0;
      if (x_dtype == W4_DTYPE_BF16)
        pf5_launch<W4_DTYPE_BF16>(p5, a, st);
      else
        pf5_launch<W4_DTYPE_FP16>(p5, a, st);
      return check_launch("w4a16_gemm (prefill, pf5)");
    }
    const Pf2Plan p = plan_pf2(M, N, K);
    if (p.ws > 0 && (ws == nullptr || ws_bytes < p.ws || (p.fin && counters == nullptr)))
      return fail(W4_ERR_WORKSPACE, "w4a16_gemm: workspace of %zu bytes required, %zu given",
                  (size_t)W4_WORKSPACE_COUNTER_BYTES + p.ws, ws ? ws_bytes : (size_t)0);
    w4::Pf2Args a{};
    a.x = static_cast<const uint16_t*>(x);
    a.qw = reinterpret_cast<const uint32_t*>(qw);
    a.sc = sc;
    a.ze = ze;
    a.y = static_cast<uint16_t*>(y);
    a.ws = p.splits > 1 ? static_cast<float*>(ws) : nullptr;
    a.sxm = sxm;
    a.ldy = ldy;
    a.x_bytes = (uint32_t)(((M - 1) * sxm + K) * 2);
    a.qw_bytes = (uint32_t)((K / 8) * N * 4);
    a.sz_bytes = (uint32_t)((K / G) * N * 2);
    a.M = (int)M;
    a.N = (int)N;
    a.K = (int)K;
    a.gshift = ilog2(G);
    a.tiles_n = p.tiles_n;
    a.tiles_mn = p.tiles_mn;
    a.kt_per_split = p.kt_per_split;
    a.cnt = p.fin ? counters : nullptr;
    a.y16 = (N % 8 == 0 && ldy % 8 == 0 && (uintptr_t)y % 16 == 0) ? 1 : 0;
    const bool szk = G < 64;
    if (x_dtype == W4_DTYPE_BF16) {
      if (p.nw == 4)
        pf2_launch_g<W4_DTYPE_BF16, 4>(p, szk, a, st);
      else
        pf2_launch_g<W4_DTYPE_BF16, 2>(p, szk, a, st);
    } else {
      if (p.nw == 4)
        pf2_launch_g<W4_DTYPE_FP16, 4>(p, szk, a, st);
      else
        pf2_launch_g<W4_DTYPE_FP16, 2>(p, szk, a, st);
    }
    int rc = check_launch("w4a16_gemm (prefill)");
    if (rc != W4_OK || p.splits == 1 || p.fin) return rc;
    return w4_splitk_reduce_launch(static_cast<const float*>(ws), p.splits, M, N, x_dtype, y, ldy, st);
  }
  // strided / unaligned activations: the general tile kernel
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

namespace {

template <int DT, int NW, int MB, int KH = 1>
void pf3_grouped_go(bool szk, const w4::Pf3Grouped& g, int wgs, hipStream_t st) {
  const dim3 grid((unsigned)wgs), block(NW * KH * 64);
  if (szk)
    hipLaunchKernelGGL((w4::pf3_grouped_kernel<DT, NW, true, MB, KH>), grid, block, 0, st, g);
  else
    hipLaunchKernelGGL((w4::pf3_grouped_kernel<DT, NW, false, MB, KH>), grid, block, 0, st, g);
}

template <int DT>
void pf3_grouped_dt(const Pf2Plan& p, bool szk, const w4::Pf3Grouped& g, int wgs, hipStream_t st) {
  if (p.nw == 4 && p.mb == 1 && p.kh == 2) {
    pf3_grouped_go<DT, 4, 1, 2>(szk, g, wgs, st);
  } else if (p.nw == 4) {
    if (p.mb == 4) pf3_grouped_go<DT, 4, 4>(szk, g, wgs, st);
    else if (p.mb == 2) pf3_grouped_go<DT, 4, 2>(szk, g, wgs, st);
    else pf3_grouped_go<DT, 4, 1>(szk, g, wgs, st);
  } else {
    if (p.mb == 4) pf3_grouped_go<DT, 2, 4>(szk, g, wgs, st);
    else if (p.mb == 2) pf3_grouped_go<DT, 2, 2>(szk, g, wgs, st);
    else pf3_grouped_go<DT, 2, 1>(szk, g, wgs, st);
  }
}

}  // namespace

// Products that share one dense activation matrix x[M, K] (same pointer, K
// and group size; x rows of K elements), as one launch of the pipelined
// kernel.  The tiling is the one the planner picks for the concatenated
// output width; plans that would split K are left to separate launches.
// Returns W4_ERR_UNSUPPORTED (nothing launched, no message) when the problems
// do not qualify.
int w4_prefill_grouped_launch(const w4a16_problem* problems, int count, int x_dtype, int64_t M, hipStream_t st) {
  if (count < 2 || count > w4::PF3_MAX_GROUPED || M < 1) return W4_ERR_UNSUPPORTED;
  const w4a16_problem& q0 = problems[0];
  const int64_t K = q0.K, G = q0.group_size;
  int64_t Nt = 0;
  for (int i = 0; i < count; ++i) {
    const w4a16_problem& q = problems[i];
    if (q.x != q0.x || q.K != K || q.group_size != G || K % w4::PF2_BK != 0 ||
        !pf2_ok(q.x, M, q.N, K, K, 1, q.qweight, q.scales, q.zeros, q.y, q.N))
      return W4_ERR_UNSUPPORTED;
    Nt += q.N;
  }
  // one launch without split-K (the tiles of all problems side by side) when
  // the model puts it below the separate launches with their own plans
  double t_grouped = 0.0, t_separate = 0.0;
  const Pf2Plan p = plan_pf2(M, Nt, K, 1, &t_grouped);
  for (int i = 0; i < count; ++i) {
    double ti = 0.0;
    plan_pf2(M, problems[i].N, K, 8, &ti);
    t_separate += ti;
  }
  if (!(t_grouped <= t_separate)) return W4_ERR_UNSUPPORTED;
  w4::Pf3Grouped g{};
  const int64_t bm = 32 * p.mb;
  const int64_t tm = (M + bm - 1) / bm;
  int wgs = 0;
  for (int i = 0; i < count; ++i) {
    const w4a16_problem& q = problems[i];
    w4::Pf2Args& a = g.prob[i];
    a.x = static_cast<const uint16_t*>(q.x);
    a.qw = reinterpret_cast<const uint32_t*>(q.qweight);
    a.sc = q.scales;
    a.ze = q.zeros;
    a.y = static_cast<uint16_t*>(q.y);
    a.ws = nullptr;
    a.sxm = K;
    a.ldy = q.N;
    a.x_bytes = (uint32_t)(M * K * 2);
    a.qw_bytes = (uint32_t)((K / 8) * q.N * 4);
    a.sz_bytes = (uint32_t)((K / G) * q.N * 2);
    a.M = (int)M;
    a.N = (int)q.N;
    a.K = (int)K;
    a.gshift = ilog2(G);
    a.tiles_n = (int)((q.N + 64 * p.nw - 1) / (64 * p.nw));
    a.tiles_mn = (int)(tm * a.tiles_n);
    a.kt_per_split = (int)(K / w4::PF2_BK);
    a.y16 = (q.N % 8 == 0 && (uintptr_t)q.y % 16 == 0) ? 1 : 0;
    g.wg_start[i] = wgs;
    wgs += a.tiles_mn;
  }
  for (int i = count; i <= w4::PF3_MAX_GROUPED; ++i) g.wg_start[i] = wgs;
  g.count = count;
  const bool szk = G < 64;
  if (x_dtype == W4_DTYPE_BF16)
    pf3_grouped_dt<W4_DTYPE_BF16>(p, szk, g, wgs, st);
  else
    pf3_grouped_dt<W4_DTYPE_FP16>(p, szk, g, wgs, st);
  return check_launch("w4a16_gemm_grouped (prefill)");
}
