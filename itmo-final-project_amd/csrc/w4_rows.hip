// Several-row W4A16 products (49 <= M <= 64, the grouped launch) for gfx950:
// every weight is dequantized once, for all M rows.
//
// Each packed word is turned into the reference's own weights (fp32
// (q - z) s rounded once to the activation dtype, int4_triton/gemm.py:139,147;
// dequant_word) and fed as the B operand of v_mfma_f32_16x16x32_{bf16,f16}
// against 64 activation rows (4 row blocks of 16).  Against the sixteen-row
// slices of the decode kernels, which dequantize a weight once per slice
// (four times at M = 64), this does the VALU work once per weight while the
// matrix cores, with all rows real, do the rest.  The host takes it for
// grouped launches of 49 <= M <= 64 rows that fill most of the chip only
// (the 7-linear decoder block in one call): there it measured faster than
// the slices (the 7-linear block at M = 64: 24.5 against 28.5 us); at 48
// rows and below, and for lone products, the slices were faster (a
// workgroup's run is a chain of memory latencies, and a K split finished by
// the last part costs about 5 us of round trips).
//
// Work decomposition (this library's own; the reference's small-M path is
// the split-K kernel of int4_triton/gemm.py:74-157 plus the reduce of
// :171-182):
//  * Column tiles of 128 columns; the K range of a tile is cut into `ksplit`
//    parts (one workgroup each).  A workgroup's eight waves are two 64-column
//    halves x four K runs of `wave_steps` steps of 32 k.  A lane owns 4
//    adjacent columns (one 16-byte load per qweight row) and one of the 4
//    qweight rows of a step; the two waves of a run read the two halves of
//    the same qweight rows, i.e. 512-byte pieces.
//  * A wave issues the loads of every packed word of its run at once (at
//    most 16 KB per wave, the workgroup's whole weight tile in flight), then
//    streams the activation block of each step (MR rows x 32 k, straight
//    from memory to the wave's own LDS slot with direct-to-LDS loads) and
//    its scales and zeros through a ring of kRowsRing steps.  Waves never
//    wait for each other until the end.
//  * The 4 per-run partial tiles of a half (MR x 64 fp32, in the LDS the
//    rings held) are summed in run order; with ksplit > 1 each part
//    publishes its tile and the last part to arrive sums all parts in part
//    order and writes y.
//  Every summation order is a function of the shapes, so results are
//  bit-identical from run to run.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <type_traits>

#include "w4_common.hpp"

namespace w4 {

struct RowsArgs {
  const uint16_t* x;
  const uint32_t* qw;
  const uint16_t* sc;
  const uint16_t* ze;
  uint16_t* y;
  int64_t sxm;        // x row stride (elements, multiple of 8)
  int64_t ldy;        // y row stride (elements, multiple of 4)
  uint32_t qw_bytes;  // loads at or past these byte offsets read 0
  uint32_t sz_bytes;
  uint32_t x_bytes;
  int N, K, M;
  int gshift;      // log2(group size), >= 5
  int ksplit;      // K parts per column tile, a power of two <= kMaxRowsSplit
  int wave_steps;  // steps of 32 k per wave: K / (ksplit * kRowsKWaves * 32)
  // ksplit > 1: one arrival counter per column tile (zero on entry, left
  // zero) and partial tiles [column tile][ksplit][MR x 128] floats
  unsigned* cnt;
  float* part;
};

struct RowsGroupedArgs {
  RowsArgs prob[W4_MAX_GROUPED];
  int wg_start[W4_MAX_GROUPED + 1];
  int count;
};

constexpr int kRowsKWaves = 4;  // waves splitting the K part of a column half
constexpr int kRowsHalves = 2;  // 64-column halves of a workgroup's tile
constexpr int kRowsWaves = kRowsKWaves * kRowsHalves;
constexpr int kRowsTile = 64 * kRowsHalves;  // columns of a workgroup
constexpr int kRowsRing = 4;           // activation / scale steps in flight per wave
constexpr int kRowsMaxWaveSteps = 16;  // steps of 32 k per wave (packed words all in flight)
constexpr int kMaxRowsSplit = 8;
constexpr int kRowsMinM = 49;  // fewer rows: the decode kernel's 16-row slices
constexpr uint32_t kRowsOOB = 0x80000000u;  // offset the buffer range check rejects
constexpr int kRowsBufFlags = 0x00020000;   // raw buffer, 32-bit data format
constexpr int kRowsStreamAux = 2;           // nt: the packed words are read once per call
constexpr int kRowsCoherentAux = 16;        // sc1: the cache policy of agent-scope atomic loads and stores

__device__ __forceinline__ void rows_lds_load16(__amdgpu_buffer_rsrc_t r, uint8_t* lds, uint32_t voffset) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (__attribute__((address_space(3))) void*)lds, 16, voffset, 0, 0, 0);
}

// 16-byte LDS read the compiler does not see as one: it would otherwise make
// every read of the ring wait for the newest direct-to-LDS load (it cannot
// tell the slots apart where a loop's iterations meet), draining the ring
// once per loop iteration.  The caller waits for the direct-to-LDS loads it
// needs (vmcnt) before, and for the reads (lgkmcnt) after.
template <int I, int E, typename Fn>
__device__ __forceinline__ void rows_static_for(Fn&& f) {
  if constexpr (I < E) {
    f(std::integral_constant<int, I>{});
    rows_static_for<I + 1, E>(f);
  }
}

template <int OFF>
__device__ __forceinline__ u32x4 rows_lds_read16(uint32_t lds_addr) {
  static_assert(OFF >= 0 && OFF < 65536, "ds offset field");
  u32x4 v;
  asm volatile("ds_read_b128 %0, %1 offset:%2" : "=v"(v) : "v"(lds_addr), "i"(OFF) : "memory");
  return v;
}

template <int DT, int MR>
__device__ __forceinline__ void rows_tile(const RowsArgs& a, const int tile, uint8_t* smem, unsigned* arrived) {
  typedef typename Act<DT>::frag F;
  static_assert(MR == 64, "the host launches 64-row tiles only");
  constexpr int RB = MR / 16;                  // row blocks of 16
  constexpr int SLOT = MR * 64;                // bytes of a step's activations: MR rows x 32 k
  constexpr int WAVE_LDS = kRowsRing * SLOT;   // one wave's ring = its MR x 64 fp32 partial tile
  constexpr int LPX = RB + 2;                  // ring loads per step: activations, scales, zeros

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wv = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int ks = a.ksplit;
  const int ks_log = __builtin_ctz((unsigned)ks);
  const int ct = tile >> ks_log;
  const int kp = tile - (ct << ks_log);
  // wave wv: column half wv % kRowsHalves (neighbouring waves read the two
  // halves of the same qweight rows at about the same time: 512-byte pieces),
  // K run wv / kRowsHalves of the part
  const int ch = wv % kRowsHalves, kq = wv / kRowsHalves;
  const int n0 = ct * kRowsTile;
  const int n0w = n0 + 64 * ch;
  const int N = a.N;
  const int S = a.wave_steps;
  const int st0 = (kp * kRowsKWaves + kq) * S;  // first step (of 32 k) of this wave
  const int lq = lane & 15, lr = lane >> 4;    // column quad, qweight row within a step
  const uint32_t gmask = (1u << a.gshift) - 1u;

  const __amdgpu_buffer_rsrc_t rx = __builtin_amdgcn_make_buffer_rsrc((void*)a.x, (short)0, (int)a.x_bytes, kRowsBufFlags);
  const __amdgpu_buffer_rsrc_t rq = __builtin_amdgcn_make_buffer_rsrc((void*)a.qw, (short)0, (int)a.qw_bytes, kRowsBufFlags);
  const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc((void*)a.sc, (short)0, (int)a.sz_bytes, kRowsBufFlags);
  const __amdgpu_buffer_rsrc_t rz = __builtin_amdgcn_make_buffer_rsrc((void*)a.ze, (short)0, (int)a.sz_bytes, kRowsBufFlags);

  // Columns past N (a partial last tile; N % 4 == 0, so a lane's four are all
  // inside or all past the end) take an offset the range check rejects: they
  // read zeros and are never stored.
  const uint32_t col_oob = n0w + 4 * lq < N ? 0u : kRowsOOB;
  const uint32_t w_lane = ((uint32_t)lr * (uint32_t)N + (uint32_t)(n0w + 4 * lq)) * 4u;  // + 16 N per step
  const uint32_t sz_lane = (uint32_t)(n0w + 4 * lq) * 2u;                                // + 2 N per group
  // Activation loads of a step: instruction j fills bytes [1024 j, +1024) of
  // the slot, lane l the 16 bytes at 1024 j + 16 l: row 16 j + l / 4 of the
  // block, 16-byte position l % 4 of that row, which holds k chunk
  // (l % 4) ^ ((row / 2) % 4).  An A-fragment read (16 rows, one chunk) then
  // covers eight distinct 16-byte bank positions per eight lanes.
  uint32_t x_lane[RB];
#pragma unroll
  for (int j = 0; j < RB; ++j) {
    const int row = 16 * j + (lane >> 2);
    const int c = (lane & 3) ^ ((lane >> 3) & 3);
    x_lane[j] = row < a.M ? ((uint32_t)row * (uint32_t)a.sxm + (uint32_t)c * 8u) * 2u : kRowsOOB;
  }
  // A fragment of row block rb: row 16 rb + l % 16, k chunk l / 16
  const uint32_t a_off = (uint32_t)(lq * 64 + ((lr ^ ((lq >> 1) & 3)) * 16));
  uint8_t* const ring = smem + wv * WAVE_LDS;
  const uint32_t magic = fp16_magic_vgpr();

  // LDS address of this lane's A fragments in the ring (slot and row block
  // come as immediate offsets)
  const uint32_t a_lds = (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) uint8_t*)ring + a_off;
  struct SZ {
    u32x2 s, z;
  };
  // Ring loads of step i (0-based) of this wave into slot SL = i % kRowsRing:
  // the activation block (direct to LDS), the scales and zeros.  Steps past
  // the run (the ring's prefetches at its end) read zeros with no memory
  // access.
  auto issue_ring = [&](SZ& r, int i, auto SL) {
    const uint32_t oob = i < S ? 0u : kRowsOOB;  // scalar
    const int st = st0 + min(i, S - 1);
    uint8_t* slot = ring + decltype(SL)::value * SLOT;
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int j = 0; j < RB; ++j) rows_lds_load16(rx, slot + 1024 * j, (x_lane[j] + (uint32_t)st * 64u) | oob);
    const uint32_t so = (((uint32_t)(st * 32) >> a.gshift) * (uint32_t)N * 2u + sz_lane) | col_oob | oob;
    r.s = __builtin_amdgcn_raw_buffer_load_b64(rs, so, 0, 0);  // a group's row is read by each of its steps
    r.z = __builtin_amdgcn_raw_buffer_load_b64(rz, so, 0, 0);
    __builtin_amdgcn_sched_barrier(0);
  };

  f32x4 acc[RB][4];
#pragma unroll
  for (int rb = 0; rb < RB; ++rb)
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[rb][j] = f32x4{0.f, 0.f, 0.f, 0.f};
  GroupConst gc[4];

  // Issue order: the ring's first kRowsRing steps, then the packed words of
  // every step of the run (all in flight at once: kRowsMaxWaveSteps x 1 KB per
  // wave), then one ring step per step computed.  Loads complete in issue
  // order, so the wait before step i is a count of the loads issued after the
  // ones it needs.
  SZ szr[kRowsRing];
  issue_ring(szr[0], 0, std::integral_constant<int, 0>{});
  issue_ring(szr[1], 1, std::integral_constant<int, 1>{});
  issue_ring(szr[2], 2, std::integral_constant<int, 2>{});
  issue_ring(szr[3], 3, std::integral_constant<int, 3>{});
  static_assert(kRowsRing == 4, "four ring slots");
  u32x4 w[kRowsMaxWaveSteps];
  __builtin_amdgcn_sched_barrier(0);
#pragma unroll
  for (int i = 0; i < kRowsMaxWaveSteps; ++i) {
    const uint32_t oob = i < S ? 0u : kRowsOOB;
    const int st = st0 + min(i, S - 1);
    w[i] = __builtin_amdgcn_raw_buffer_load_b128(rq, (w_lane + (uint32_t)st * 16u * (uint32_t)N) | col_oob | oob, 0,
                                                 kRowsStreamAux);
  }
  __builtin_amdgcn_sched_barrier(0);

  rows_static_for<0, kRowsMaxWaveSteps>([&](auto I) {
    constexpr int i = decltype(I)::value;
    constexpr int SL = i % kRowsRing;
    constexpr int SO = SL * SLOT;
    // loads issued after the ones step i needs: for the ring's first steps,
    // the packed words after its own and the ring steps issued so far; later,
    // the ring steps i + 1 .. i + kRowsRing - 1
    constexpr int AFTER = i < kRowsRing ? (kRowsMaxWaveSteps - 1 - i) + i * LPX : (kRowsRing - 1) * LPX;
    static_assert(AFTER < 64, "vmcnt range");
    constexpr int WAIT_IMM = (AFTER & 15) | 0x70 | 0xF00 | ((AFTER >> 4) << 14);
    if (i < S) {  // uniform
      __builtin_amdgcn_sched_barrier(0);
      __builtin_amdgcn_s_waitcnt(WAIT_IMM);
      asm volatile("" ::: "memory");
      __builtin_amdgcn_sched_barrier(0);
      u32x4 ar[RB];
      ar[0] = rows_lds_read16<SO>(a_lds);
      ar[1] = rows_lds_read16<SO + 1024>(a_lds);
      ar[2] = rows_lds_read16<SO + 2048>(a_lds);
      ar[3] = rows_lds_read16<SO + 3072>(a_lds);
      // the reads' results are tied to the wait, so no use moves above it
      asm volatile("s_waitcnt lgkmcnt(0)" : "+v"(ar[0]), "+v"(ar[1]), "+v"(ar[2]), "+v"(ar[3]));
      const SZ& r = szr[SL];
      if (i == 0 || (((uint32_t)(st0 + i) * 32u) & gmask) == 0) {  // first step of a group (uniform)
#pragma unroll
        for (int j = 0; j < 4; ++j)
          gc[j] = make_group_const((uint16_t)(r.s[j >> 1] >> (16 * (j & 1))), (uint16_t)(r.z[j >> 1] >> (16 * (j & 1))));
      }
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const F b = dequant_word<DT>(w[i][j], gc[j], magic);
#pragma unroll
        for (int rb = 0; rb < RB; ++rb) acc[rb][j] = Mfma<DT>::m16(__builtin_bit_cast(F, ar[rb]), b, acc[rb][j]);
      }
      __builtin_amdgcn_sched_barrier(0);
      issue_ring(szr[SL], i + kRowsRing, std::integral_constant<int, SL>{});
    }
  });
  __builtin_amdgcn_s_waitcnt(0);  // the ring's trailing loads have written their slots
  asm volatile("" ::: "memory");

  // The wave's partial tile, row-major MR x 64 fp32, over its own ring:
  // accumulator element r of block (rb, j) is row 16 rb + 4 lr + r, column
  // 4 lq + j.
  float* const red = reinterpret_cast<float*>(smem);
#pragma unroll
  for (int rb = 0; rb < RB; ++rb)
#pragma unroll
    for (int r = 0; r < 4; ++r)
      *reinterpret_cast<f32x4*>(&red[wv * (MR * 64) + (16 * rb + 4 * lr + r) * 64 + 4 * lq]) =
          f32x4{acc[rb][0][r], acc[rb][1][r], acc[rb][2][r], acc[rb][3][r]};
  __syncthreads();

  // Thread tid sums quads q = tid + 64 kRowsWaves u of the workgroup's tile
  // (row q / 32, columns 4 (q % 32) .. + 3: half (q % 32) / 16) over the K
  // runs of that half in run order.
  constexpr int QPR = kRowsTile / 4;                   // quads per tile row
  constexpr int QPT = MR * QPR / (kRowsWaves * 64);  // quads per thread
  f32x4 v[QPT];
#pragma unroll
  for (int u = 0; u < QPT; ++u) {
    const int q = tid + u * kRowsWaves * 64;
    const int row = q / QPR, cq = q % QPR;
    const float* base = red + (cq / 16) * (MR * 64) + row * 64 + 4 * (cq % 16);
    f32x4 pv[kRowsKWaves];
#pragma unroll
    for (int r = 0; r < kRowsKWaves; ++r) pv[r] = *reinterpret_cast<const f32x4*>(base + r * kRowsHalves * (MR * 64));
    v[u] = pv[0];
#pragma unroll
    for (int r = 1; r < kRowsKWaves; ++r) v[u] += pv[r];
  }
  if (ks > 1) {
    // Publish this part's tile, wait until the stores have completed, count
    // the arrival; the last part sums every part in part order (so the result
    // does not depend on which part is last), writes y and leaves the counter
    // at zero.  The tiles move as 128-bit buffer accesses with the sc1 policy,
    // the one the compiler gives agent-scope atomic loads and stores (written
    // through to, and read from, the level all XCDs share); their order
    // against the arrival counter comes from the waits and barriers, as for
    // atomics.
    constexpr int E = MR * kRowsTile;
    float* const tiles = a.part + (int64_t)ct * ks * E;
    const __amdgpu_buffer_rsrc_t rp =
        __builtin_amdgcn_make_buffer_rsrc((void*)tiles, (short)0, ks * E * (int)sizeof(float), kRowsBufFlags);
#pragma unroll
    for (int u = 0; u < QPT; ++u) {
      const int q = tid + u * kRowsWaves * 64;
      // (the whole vector is bit-cast: a bit cast of one element of an
      // ext_vector_type value reads the vector's first element)
      __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, v[u]), rp, (uint32_t)(kp * E + 4 * q) * 4u, 0,
                                             kRowsCoherentAux);
    }
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    if (tid == 0) *arrived = __hip_atomic_fetch_add(a.cnt + ct, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    __syncthreads();
    if (*arrived != (unsigned)(ks - 1)) return;
    if (tid == 0) __hip_atomic_store(a.cnt + ct, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    // every part's tile is requested before the first add
    u32x4 other[QPT][kMaxRowsSplit];
#pragma unroll
    for (int u = 0; u < QPT; ++u) {
      const int q = tid + u * kRowsWaves * 64;
#pragma unroll
      for (int p = 0; p < kMaxRowsSplit; ++p)
        if (p < ks && p != kp)
          other[u][p] = __builtin_amdgcn_raw_buffer_load_b128(rp, (uint32_t)(p * E + 4 * q) * 4u, 0, kRowsCoherentAux);
    }
#pragma unroll
    for (int u = 0; u < QPT; ++u) {
      f32x4 sum = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int p = 0; p < kMaxRowsSplit; ++p) {
        if (p < ks) {
          const f32x4 t = p == kp ? v[u] : __builtin_bit_cast(f32x4, other[u][p]);
          sum = p == 0 ? t : sum + t;
        }
      }
      v[u] = sum;
    }
  }
#pragma unroll
  for (int u = 0; u < QPT; ++u) {
    const int q = tid + u * kRowsWaves * 64;
    const int m = q / QPR, n = n0 + 4 * (q % QPR);
    if (m < a.M && n < N) {
      const u32x2 o = u32x2{(uint32_t)float_to_act_bits<DT>(v[u][0]) | ((uint32_t)float_to_act_bits<DT>(v[u][1]) << 16),
                            (uint32_t)float_to_act_bits<DT>(v[u][2]) | ((uint32_t)float_to_act_bits<DT>(v[u][3]) << 16)};
      *reinterpret_cast<u32x2*>(a.y + (int64_t)m * a.ldy + n) = o;
    }
  }
}

template <int DT, int MR>
__global__ __launch_bounds__(64 * kRowsWaves) __attribute__((amdgpu_waves_per_eu(2))) void rows_kernel(
    RowsGroupedArgs g) {
  __shared__ __attribute__((aligned(16))) uint8_t smem[kRowsWaves * kRowsRing * MR * 64];
  __shared__ unsigned arrived;
  // Workgroups go to the 8 XCDs round-robin by index; XCD x takes the x-th
  // contiguous run of the tile order instead, so each XCD works on one to
  // three problems and its L2 fetches only their activation blocks (at
  // M = 64 each is 256 KB to 1 MB and is read by every column tile).
  const int W = g.wg_start[W4_MAX_GROUPED];
  const int q8 = W >> 3, r8 = W & 7;
  const int xcd = (int)blockIdx.x & 7;
  const int t = xcd * q8 + min(xcd, r8) + ((int)blockIdx.x >> 3);
  int p = 0;
#pragma unroll
  for (int i = 1; i < W4_MAX_GROUPED; ++i)
    if (i < g.count && t >= g.wg_start[i]) p = i;
  rows_tile<DT, MR>(g.prob[p], t - g.wg_start[p], smem, &arrived);
}

}  // namespace w4

using namespace w4host;

namespace {

struct RowsPlan {
  w4::RowsGroupedArgs g;
  int wgs;
  int mr;
  int64_t cnt_words, part_floats;
  int64_t cnt_off[W4_MAX_GROUPED], part_off[W4_MAX_GROUPED];
};

// Launch table: a pure function of shapes, strides and pointer alignment.
// Returns false (nothing to launch) when a problem does not fit: group size
// < 32, K not a multiple of 128, N not a multiple of 4, misaligned or
// non-dense operands, or offsets past 2 GiB.
//
// K parts: at most 2048 k per workgroup (16 steps per wave).  (Halving them
// further to fill the chip cost more than it gained: every split problem
// pays the last part's round trips.)
bool rows_plan(const w4a16_problem* problems, const int64_t* sxm, const int64_t* ldy, int count, int64_t M,
               RowsPlan& rp) {
  rp = RowsPlan{};
  if (count < 1 || count > W4_MAX_GROUPED || M < w4::kRowsMinM || M > 64) return false;
  const int mr = 64;
  int ks[W4_MAX_GROUPED];
  for (int i = 0; i < count; ++i) {
    const w4a16_problem& q = problems[i];
    const int64_t G = q.group_size, N = q.N, K = q.K;
    const int64_t ly = ldy != nullptr ? ldy[i] : N;
    if (G < 32 || !is_pow2(G) || K % G != 0 || K % 128 != 0 || N < 4 || N % 4 != 0) return false;
    if (N >= (1LL << 27) || K >= (1LL << 30) || (K / 8) * N * 4 >= (1LL << 31)) return false;
    if (((uintptr_t)q.x % 16) != 0 || ((uintptr_t)q.qweight % 16) != 0 || ((uintptr_t)q.scales % 8) != 0 ||
        ((uintptr_t)q.zeros % 8) != 0 || ((uintptr_t)q.y % 8) != 0)
      return false;
    if (sxm[i] % 8 != 0 || sxm[i] < K || ((M - 1) * sxm[i] + K) * 2 >= (1LL << 31)) return false;
    if (ly < N || ly % 4 != 0) return false;
    int k = 1;
    while (K / k > (int64_t)w4::kRowsKWaves * 32 * w4::kRowsMaxWaveSteps) k *= 2;  // 2048
    if (k > w4::kMaxRowsSplit || K % (128 * k) != 0) return false;
    ks[i] = k;
  }
  // longest-running workgroups first
  int order[W4_MAX_GROUPED];
  for (int i = 0; i < count; ++i) order[i] = i;
  std::stable_sort(order, order + count,
                   [&](int l, int r) { return problems[l].K / ks[l] > problems[r].K / ks[r]; });
  int wgs = 0;
  for (int s = 0; s < count; ++s) {
    const int i = order[s];
    const w4a16_problem& q = problems[i];
    w4::RowsArgs& a = rp.g.prob[s];
    a.x = static_cast<const uint16_t*>(q.x);
    a.qw = reinterpret_cast<const uint32_t*>(q.qweight);
    a.sc = q.scales;
    a.ze = q.zeros;
    a.y = static_cast<uint16_t*>(q.y);
    a.sxm = sxm[i];
    a.ldy = ldy != nullptr ? ldy[i] : q.N;
    a.qw_bytes = (uint32_t)((q.K / 8) * q.N * 4);
    a.sz_bytes = (uint32_t)((q.K / q.group_size) * q.N * 2);
    a.x_bytes = (uint32_t)(((M - 1) * sxm[i] + q.K) * 2);
    a.N = (int)q.N;
    a.K = (int)q.K;
    a.M = (int)M;
    a.gshift = ilog2(q.group_size);
    a.ksplit = ks[i];
    a.wave_steps = (int)(q.K / ((int64_t)ks[i] * w4::kRowsKWaves * 32));
    a.cnt = nullptr;
    a.part = nullptr;
    const int64_t tiles = (q.N + w4::kRowsTile - 1) / w4::kRowsTile;
    if (ks[i] > 1) {
      rp.cnt_off[s] = rp.cnt_words;
      rp.part_off[s] = rp.part_floats;
      rp.cnt_words += tiles;
      rp.part_floats += tiles * ks[i] * mr * w4::kRowsTile;
    }
    rp.g.wg_start[s] = wgs;
    if (tiles * ks[i] > (1 << 24)) return false;
    wgs += (int)(tiles * ks[i]);
  }
  // Fewer workgroups than three quarters of the CUs (q/k/v or gate/up alone at
  // M = 64: 24 or 128 workgroups of this kernel): the slices' many small
  // workgroups were faster (the 4-call block at M = 64: 38.6 against 51.5 us)
  if (wgs < device_cu_count() * 3 / 4) return false;
  for (int s = count; s <= W4_MAX_GROUPED; ++s) rp.g.wg_start[s] = wgs;
  rp.g.count = count;
  rp.wgs = wgs;
  rp.mr = mr;
  return wgs > 0 && rp.cnt_words * 4 <= W4_WORKSPACE_COUNTER_BYTES;
}

template <int DT>
void rows_launch(const RowsPlan& rp, hipStream_t st) {
  const dim3 grid((unsigned)rp.wgs), block(64 * w4::kRowsWaves);
  hipLaunchKernelGGL((w4::rows_kernel<DT, 64>), grid, block, 0, st, rp.g);
}

}  // namespace

// Several-row launch (17 <= M <= 64, every problem with M rows).  Returns
// W4_ERR_UNSUPPORTED, with nothing launched and no error message, when a
// problem does not fit this kernel.  sxm: activation row strides, ldy: output
// row strides (elements; null = dense).
int w4_rows_launch(const w4a16_problem* problems, const int64_t* sxm, const int64_t* ldy, int count, int x_dtype,
                   int64_t M, unsigned* counters, void* scratch, size_t scratch_bytes, hipStream_t st) {
  RowsPlan rp;
  if (!rows_plan(problems, sxm, ldy, count, M, rp)) return W4_ERR_UNSUPPORTED;
  if (rp.cnt_words > 0) {
    const size_t need = (size_t)rp.part_floats * 4;
    if (counters == nullptr || scratch == nullptr || scratch_bytes < need)
      return fail(W4_ERR_WORKSPACE, "w4a16 several-row kernel: a workspace of %zu bytes is required",
                  (size_t)W4_WORKSPACE_COUNTER_BYTES + need);
    for (int s = 0; s < rp.g.count; ++s) {
      w4::RowsArgs& a = rp.g.prob[s];
      if (a.ksplit > 1) {
        a.cnt = counters + rp.cnt_off[s];
        a.part = static_cast<float*>(scratch) + rp.part_off[s];
      }
    }
  }
  if (x_dtype == W4_DTYPE_BF16)
    rows_launch<W4_DTYPE_BF16>(rp, st);
  else
    rows_launch<W4_DTYPE_FP16>(rp, st);
  return check_launch("w4a16 several-row kernel");
}

// Workspace bytes w4_rows_launch needs (0: none, or the kernel does not take
// these problems).  Pointers are only used for their alignment.
size_t w4_rows_workspace_bytes(const w4a16_problem* problems, const int64_t* sxm, int count, int64_t M) {
  RowsPlan rp;
  if (!rows_plan(problems, sxm, nullptr, count, M, rp) || rp.cnt_words == 0) return 0;
  return W4_WORKSPACE_COUNTER_BYTES + (size_t)rp.part_floats * 4;
}
