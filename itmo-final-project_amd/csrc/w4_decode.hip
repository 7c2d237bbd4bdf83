// Decode-shaped W4A16 products (1 <= M <= 16, group size >= 32; up to 128
// rows as 16-row slices of one launch) for gfx950: one launch, no reduce
// launch, the dequantization factored out of the K loop.
//
// Arithmetic.  For one output column n and one quantization group g,
//   sum_k x_k (q_k - z) s = s * ( sum_k x_k (OFF + QS q_k) - OFF xs - QS z xs ) / QS
// with xs = sum_k x_k over the group.  The matrix core computes the first sum
// on raw nibbles: each nibble is inserted into the mantissa of a 16-bit float
// whose exponent is fixed, which gives OFF + QS*q exactly (bf16: 0x4300|q =
// 128 + q; fp16: 0x6400|(q << 6) = 1024 + 64 q) with one v_and_or_b32 per two
// nibbles.  xs comes from one more MFMA against a vector of ones.  The scale
// and zero point are applied once per group and column in fp32 (three fused
// multiply-adds), so the per-weight work is 7 (bf16) or 8 (fp16) VALU
// instructions per packed word instead of a full dequantization.  W_hat is
// never rounded to the activation dtype: the result is x @ W_hat^T with the
// exact fp32 W_hat = (q - z) * s, accumulated in fp32 (the reference rounds
// W_hat to the activation dtype first, int4_triton/gemm.py:139,203; both are
// within the reference's tolerance of the exact product).
//
// Two kernels.  dec_kernel_one (further down) takes every launch whose
// operands are 16-byte aligned with N % 8 == 0: one workgroup of 16 waves per
// CU-sized tile, all loads of a wave in flight at once, K longer than its
// single-round tilings cut into K parts combined across workgroups (a pair
// tree of compare-and-swap words at M = 1, the last part to arrive for more
// rows).  dec_kernel, the generic kernel, takes the rest:
//
// Work decomposition (dec_kernel).  A workgroup owns a column tile of
// TN = 16*VEC columns over the whole K (no cross-workgroup reduction).
// VEC = 4 (256-byte row segments) for K <= 4096, VEC = 2 (128-byte segments,
// one cache line) for longer K, so a workgroup streams at most 128 KB for
// K <= 8192.  Its eight waves take contiguous runs of 32-wide K steps and
// stream them in chunks of C steps, double buffered: the next chunk's
// weights, activations and scales/zeros are in flight while the current one
// is computed.  All loads are raw buffer loads; a chunk past the end of a
// wave's run uses an offset that the hardware range check turns into zeros
// with no memory traffic, so the load sequence is unconditional.  The
// per-wave partial tiles are summed through LDS in wave order, so every
// output bit is fixed.
//
// Nibble order.  The four dwords built from one packed word hold nibbles
// (0,4), (1,5), (2,6), (3,7); the activation fragment is permuted to the same
// k order with four v_perm_b32, so the dot product is unchanged.
#include <hip/hip_runtime.h>

#include <algorithm>

#include "w4_common.hpp"

namespace w4 {

struct DecArgs {
  const uint16_t* x;
  const uint32_t* qw;
  const uint16_t* sc;
  const uint16_t* ze;
  uint16_t* y;
  int64_t sxm;        // x row stride in elements (multiple of 8)
  int64_t ldy;        // y row stride in elements
  uint32_t qw_bytes;  // loads at or past these byte offsets read 0
  uint32_t sz_bytes;
  uint32_t x_bytes;
  int N, K, M;
  int gshift;  // log2(group size), >= 5
  int vec;     // generic path: columns per lane, 4, 2 or 1
  int cfg;     // M == 1: kCfg* tiling of dec_kernel_one
  // M == 1, dec_kernel_one: K parts per column tile (a power of two).  1: the
  // workgroup covers all of K and writes y.  > 1: workgroup t covers part
  // t % ksplit of column tile t / ksplit; the parts of a column meet pairwise
  // in a fixed binary tree of 64-bit words `pair` [tile][ksplit - 1][TW]
  // (zero on entry and left zero), see dec_split_finish.
  int ksplit;
  unsigned long long* pair;
  // 16-row launches: M may exceed 16; the problem is then cut into `slices`
  // row slices of 16, workgroup t covering column tile (and K part)
  // t % col_tiles of slice t / col_tiles (dec_kernel_slices; dec_kernel via
  // dec_row_slice).
  // dec_kernel: workgroup t covers column tile t % col_tiles of rows
  // [16 s, 16 s + 16), s = t / col_tiles (see dec_row_slice).
  int slices;
  int col_tiles;
  // M > 1, ksplit > 1: per column tile one arrival counter (zero on entry
  // and left zero) and ksplit partial tiles of MR x 64 floats (MR = the
  // launch's row count: 4, 8 or 16)
  unsigned* cnt;
  float* part;
};

// The column tile and row slice of tile `tile` of a 16-row problem: a copy of
// the problem's arguments with x, y, M and the activation range narrowed to the
// slice.  Slice-major order keeps the slices of one column tile on one XCD
// when col_tiles is a multiple of 8 (workgroups go to the XCDs round-robin),
// so their reads of the same weights meet in that XCD's L2.
__device__ __forceinline__ DecArgs dec_row_slice(const DecArgs& g, int& tile) {
  DecArgs a = g;
  if (g.slices > 1) {
    const int s = tile / g.col_tiles;
    tile -= s * g.col_tiles;
    const int r0 = 16 * s;
    a.x = g.x + (int64_t)r0 * g.sxm;
    a.y = g.y + (int64_t)r0 * g.ldy;
    a.M = min(16, g.M - r0);
    a.x_bytes = (uint32_t)(((int64_t)(a.M - 1) * g.sxm + g.K) * 2);
    if (g.ksplit > 1) {
      a.cnt = g.cnt + (int64_t)s * (g.col_tiles / g.ksplit);
      a.part = g.part + (int64_t)s * g.col_tiles * (16 * 64);
    }
  }
  return a;
}

// M == 1 tilings (dec_kernel_one)
constexpr int kCfgT128 = 0;     // 128 columns, one round of 8 loads per wave (K <= 2048)
constexpr int kCfgT64 = 1;      // 64 columns, one round (K <= 4096)
constexpr int kCfgT64Ring = 2;  // 64 columns, rounds of 4 loads, two in flight (group 32, long K)
constexpr int kCfgT32 = 3;      // 32 columns, one round (K <= 8192)
constexpr int kCfgT32Ring = 4;  // 32 columns, rounds of 4 loads, two in flight (K > 8192)

struct DecGroupedArgs {
  DecArgs prob[W4_MAX_GROUPED];
  int wg_start[W4_MAX_GROUPED + 1];
  int count;
};

constexpr int kDecWaves = 8;
constexpr int kDecThreads = 64 * kDecWaves;
constexpr uint32_t kDecOOB = 0x80000000u;  // offset the buffer range check rejects
constexpr int kDecBufFlags = 0x00020000;   // raw buffer, 32-bit data format
// Cache policy of the packed-weight loads: non-temporal (nt).  Each weight
// byte is read once per call; decode steps stream far more weights than the
// 256 MB Infinity Cache holds (a Llama-3.2-1B token reads 517 MB), and
// streaming them with nt took the rotated-weights M = 1 block from 10.2 to
// 9.6 us.  A weight set small enough to stay cache-resident between calls
// loses that reuse (6.2 -> 8.2 us per block in that case).  Scales and zeros
// are read once per call as well and take the same policy (M = 1 block
// 9.5 -> 9.2 us with both).
constexpr int kDecWeightAux = 2;
constexpr int kDecCoherentAux = 16;  // sc1: the cache policy of agent-scope atomic loads and stores

template <int DT>
struct DecNum;
template <>
struct DecNum<W4_DTYPE_BF16> {
  static constexpr float OFF = 128.0f, QS = 1.0f;
  static constexpr uint32_t ONES = 0x3F803F80u;
  static constexpr uint32_t MAGIC = 0x43004300u;
  // nibbles (i, i+4) -> 128 + q at mantissa bits 0..3 of each half
  __device__ __forceinline__ static u32x4 bvals(uint32_t w, uint32_t magic) {
    u32x4 d;
    d[0] = (w & 0x000F000Fu) | magic;
    d[1] = ((w >> 4) & 0x000F000Fu) | magic;
    d[2] = ((w >> 8) & 0x000F000Fu) | magic;
    d[3] = ((w >> 12) & 0x000F000Fu) | magic;
    return d;
  }
};
template <>
struct DecNum<W4_DTYPE_FP16> {
  static constexpr float OFF = 1024.0f, QS = 64.0f;
  static constexpr uint32_t ONES = 0x3C003C00u;
  static constexpr uint32_t MAGIC = 0x64006400u;
  // nibbles (i, i+4) -> 1024 + 64 q at mantissa bits 6..9 of each half
  __device__ __forceinline__ static u32x4 bvals(uint32_t w, uint32_t magic) {
    u32x4 d;
    d[0] = ((w << 6) & 0x03C003C0u) | magic;
    d[1] = ((w << 2) & 0x03C003C0u) | magic;
    d[2] = ((w >> 2) & 0x03C003C0u) | magic;
    d[3] = ((w >> 6) & 0x03C003C0u) | magic;
    return d;
  }
};

template <int DT>
__device__ __forceinline__ uint32_t dec_magic_vgpr() {
  // kept in a VGPR so each nibble pair costs one v_and_or_b32 (mask in an SGPR)
  uint32_t m;
  if constexpr (DT == W4_DTYPE_BF16)
    asm volatile("v_mov_b32 %0, 0x43004300" : "=v"(m));
  else
    asm volatile("v_mov_b32 %0, 0x64006400" : "=v"(m));
  return m;
}

// x[k0 .. k0+7] (dwords X0..X3 = pairs (0,1),(2,3),(4,5),(6,7)) -> the k
// order of DecNum::bvals: pairs (0,4),(1,5),(2,6),(3,7).
__device__ __forceinline__ u32x4 dec_perm_x(u32x4 v) {
  u32x4 r;
  r[0] = __builtin_amdgcn_perm(v[2], v[0], 0x05040100u);
  r[1] = __builtin_amdgcn_perm(v[2], v[0], 0x07060302u);
  r[2] = __builtin_amdgcn_perm(v[3], v[1], 0x05040100u);
  r[3] = __builtin_amdgcn_perm(v[3], v[1], 0x07060302u);
  return r;
}

template <int VEC>
struct DecW;
template <>
struct DecW<4> {
  typedef u32x4 T;
  __device__ __forceinline__ static T load(__amdgpu_buffer_rsrc_t r, uint32_t vo) {
    return __builtin_amdgcn_raw_buffer_load_b128(r, vo, 0, kDecWeightAux);
  }
  __device__ __forceinline__ static uint32_t get(const T& v, int j) { return v[j]; }
};
template <>
struct DecW<2> {
  typedef u32x2 T;
  __device__ __forceinline__ static T load(__amdgpu_buffer_rsrc_t r, uint32_t vo) {
    return __builtin_amdgcn_raw_buffer_load_b64(r, vo, 0, kDecWeightAux);
  }
  __device__ __forceinline__ static uint32_t get(const T& v, int j) { return v[j]; }
};
template <>
struct DecW<1> {
  typedef uint32_t T;
  __device__ __forceinline__ static T load(__amdgpu_buffer_rsrc_t r, uint32_t vo) {
    return __builtin_amdgcn_raw_buffer_load_b32(r, vo, 0, kDecWeightAux);
  }
  __device__ __forceinline__ static uint32_t get(const T& v, int) { return v; }
};

// fp16 bit patterns of the scales (or zeros) of VEC adjacent columns
template <int VEC>
struct DecH;
template <>
struct DecH<4> {
  u32x2 v;
  __device__ __forceinline__ void load(__amdgpu_buffer_rsrc_t r, uint32_t off) {
    v = __builtin_amdgcn_raw_buffer_load_b64(r, off, 0, 0);
  }
  __device__ __forceinline__ float get(int j) const {
    return half_bits_to_float((uint16_t)(v[j >> 1] >> (16 * (j & 1))));
  }
};
template <>
struct DecH<2> {
  uint32_t v;
  __device__ __forceinline__ void load(__amdgpu_buffer_rsrc_t r, uint32_t off) {
    v = __builtin_amdgcn_raw_buffer_load_b32(r, off, 0, 0);
  }
  __device__ __forceinline__ float get(int j) const { return half_bits_to_float((uint16_t)(v >> (16 * j))); }
};
template <>
struct DecH<1> {
  uint32_t v;
  __device__ __forceinline__ void load(__amdgpu_buffer_rsrc_t r, uint32_t off) {
    v = __builtin_amdgcn_raw_buffer_load_b16(r, off, 0, 0);
  }
  __device__ __forceinline__ float get(int) const { return half_bits_to_float((uint16_t)v); }
};

// Generic path: steps (32-wide K slices) per chunk, two chunks in flight per
// wave (4 KB of weights per chunk for VEC 4 and 2).
template <int VEC>
struct DecChunk {
  static constexpr int C = VEC == 4 ? 4 : 8;
  static constexpr int D = 2;
};

// One workgroup = one column tile over all of K.
//   ONE: M == 1.  Activations travel with each chunk (lanes 0..4C-1 load one
//        8-element k slice each), are permuted once and shared through LDS;
//        all 16 rows of the MFMA operand repeat row 0, so only element 0 of
//        each accumulator is corrected and reduced.
//   !ONE: rows 0..M-1 (M <= MX; lanes with c >= M repeat row M-1).  A
//        chunk's activations (M rows x 4C 16-byte k slices, each row a
//        contiguous 64C-byte run) travel with it as XL = MX*C/16 coalesced
//        loads per wave (entry f = 64 j + lane: row f / 4C, slice f % 4C);
//        they are permuted once and staged in the wave's own LDS area, slice
//        s of row m at slot 4C m + (s ^ m), so both the staging writes and the
//        per-step fragment reads (16 rows of one slice) are free of bank
//        conflicts.
// GS = correction interval in steps (min(group size / 32, C)).
template <int DT, int VEC, bool ONE, int GS, int MX>
__device__ __forceinline__ void dec_tile(const DecArgs& a, int tile, float* red, uint32_t* xl) {
  typedef typename Act<DT>::frag F;
  typedef DecNum<DT> Num;
  typedef typename DecW<VEC>::T WT;
  constexpr int TN = 16 * VEC;
  constexpr int C = DecChunk<VEC>::C;
  constexpr int D = DecChunk<VEC>::D;
  constexpr int NP = C / GS;  // correction points per chunk
  constexpr int R = ONE ? 1 : 4;
  constexpr int C4 = 4 * C;              // 16-byte activation slices per row and chunk
  constexpr int XL = ONE ? 1 : MX * C / 16;  // activation loads per chunk and lane
  static_assert(GS >= 1 && GS <= C && (C % GS) == 0, "correction interval");
  static_assert(ONE || (XL >= 1 && MX <= C4 && MX <= 16), "activation staging");

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wv = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform: run bounds stay scalar
  const int c = lane & 15, kb = lane >> 4;
  const int N = a.N, K = a.K, M = a.M;
  const int n0 = tile * TN;
  const int S = K >> 5;
  const int per_wave = ((S + kDecWaves - 1) / kDecWaves + C - 1) / C * C;
  const int wb = min(S, wv * per_wave);
  const int we = min(S, wb + per_wave);

  const __amdgpu_buffer_rsrc_t rq =
      __builtin_amdgcn_make_buffer_rsrc((void*)a.qw, (short)0, (int)a.qw_bytes, kDecBufFlags);
  const __amdgpu_buffer_rsrc_t rs =
      __builtin_amdgcn_make_buffer_rsrc((void*)a.sc, (short)0, (int)a.sz_bytes, kDecBufFlags);
  const __amdgpu_buffer_rsrc_t rz =
      __builtin_amdgcn_make_buffer_rsrc((void*)a.ze, (short)0, (int)a.sz_bytes, kDecBufFlags);
  const __amdgpu_buffer_rsrc_t rx =
      __builtin_amdgcn_make_buffer_rsrc((void*)a.x, (short)0, (int)a.x_bytes, kDecBufFlags);

  const uint32_t step_bytes = 16u * (uint32_t)N;  // four qweight rows
  const uint32_t col = (uint32_t)(n0 + VEC * c);
  const uint32_t w_lane = ((uint32_t)kb * (uint32_t)N + col) * 4u;
  const uint32_t sz_lane = col * 2u;
  // ONE: lane l < 4C carries k8 row 4*sb + l of the chunk
  const uint32_t x_lane = (uint32_t)lane * 16u;
  // !ONE: load j carries entry f = 64 j + lane = (row f / 4C, slice f % 4C);
  // rows >= M are out of range (no traffic), so are slices past K (zeros)
  uint32_t x_off[XL];
  int x_step[XL];
  if constexpr (!ONE) {
#pragma unroll
    for (int j = 0; j < XL; ++j) {
      const int f = 64 * j + lane;
      const int m = f / C4, sl = f % C4;
      x_step[j] = sl >> 2;
      x_off[j] = m < M ? (uint32_t)((int64_t)m * a.sxm * 2) + (uint32_t)sl * 16u : kDecOOB;
    }
  }
  // read slot of step 0 (row c, rows past M repeat row M - 1); step st adds
  // 4 st inside the XOR.  Slice s of row m sits at slot C4 m + (s ^ (m % C4)).
  const int mc = min(c, M - 1);
  const int x_rd = mc * C4 + (kb ^ (mc & (C4 - 1)));
  const uint32_t magic = dec_magic_vgpr<DT>();
  const F ones = __builtin_bit_cast(F, u32x4{Num::ONES, Num::ONES, Num::ONES, Num::ONES});

  struct Chunk {
    WT w[C];
    DecH<VEC> s[NP], z[NP];
    u32x4 xv[XL];
  };

  // Out-of-range offsets are formed by OR-ing bit 31 in (never by selecting
  // between two offsets), so the compiler keeps every load unconditional.
  // Scheduling barriers pin the issue order (activations, scales/zeros,
  // weights; chunk after chunk) to the order of use, so the waits at the loop
  // head count only the older chunk's loads.
  const uint32_t x_lane_oob = (ONE && lane >= 4 * C) ? kDecOOB : 0u;
  auto load_chunk = [&](Chunk& ch, int sb) {
    const uint32_t oob = sb < we ? 0u : kDecOOB;  // scalar
    __builtin_amdgcn_sched_barrier(0);
    if constexpr (ONE) {
      const uint32_t xo = ((uint32_t)sb * 64u + x_lane) | x_lane_oob | oob;
      ch.xv[0] = __builtin_amdgcn_raw_buffer_load_b128(rx, xo, 0, 0);
      __builtin_amdgcn_sched_barrier(0);
    } else {
#pragma unroll
      for (int j = 0; j < XL; ++j) {
        // slices of steps past K read 0 (the next row must not leak in)
        const uint32_t xoob = sb + x_step[j] < S ? oob : kDecOOB;
        ch.xv[j] = __builtin_amdgcn_raw_buffer_load_b128(rx, ((uint32_t)sb * 64u + x_off[j]) | xoob, 0, 0);
      }
      __builtin_amdgcn_sched_barrier(0);
    }
#pragma unroll
    for (int p = 0; p < NP; ++p) {
      const uint32_t g = (uint32_t)(((sb + p * GS) * 32) >> a.gshift);
      const uint32_t off = (g * (uint32_t)N * 2u + sz_lane) | oob;
      ch.s[p].load(rs, off);
      ch.z[p].load(rz, off);
    }
    __builtin_amdgcn_sched_barrier(0);
    const uint32_t vo = ((uint32_t)sb * step_bytes + w_lane) | oob;
#pragma unroll
    for (int i = 0; i < C; ++i) ch.w[i] = DecW<VEC>::load(rq, vo + (uint32_t)i * step_bytes);
    __builtin_amdgcn_sched_barrier(0);
  };

  f32x4 acc[VEC];
  f32x4 xs;
  float tot[VEC][R];
#pragma unroll
  for (int j = 0; j < VEC; ++j)
#pragma unroll
    for (int r = 0; r < R; ++r) tot[j][r] = 0.0f;

  auto compute_chunk = [&](const Chunk& ch) {
    if constexpr (ONE) {
      // share this chunk's activations: slot l holds k8 row 4*sb + l, permuted
      const u32x4 v = dec_perm_x(ch.xv[0]);
      *reinterpret_cast<u32x4*>(xl + (wv * 64 + lane) * 4) = v;
      __builtin_amdgcn_wave_barrier();
    } else {
      // stage this chunk's activations in the wave's area, permuted
#pragma unroll
      for (int j = 0; j < XL; ++j) {
        const int f = 64 * j + lane;
        const int m = f / C4, sl = f % C4;
        *reinterpret_cast<u32x4*>(xl + (wv * MX * C4 + m * C4 + (sl ^ (m & (C4 - 1)))) * 4) =
            dec_perm_x(ch.xv[j]);
      }
      __builtin_amdgcn_wave_barrier();
    }
#pragma unroll
    for (int p = 0; p < NP; ++p) {
#pragma unroll
      for (int i = 0; i < GS; ++i) {
        const int st = p * GS + i;
        F xa;
        if constexpr (ONE)
          xa = __builtin_bit_cast(F, *reinterpret_cast<const u32x4*>(xl + (wv * 64 + st * 4 + kb) * 4));
        else
          xa = __builtin_bit_cast(F, *reinterpret_cast<const u32x4*>(xl + (wv * MX * C4 + (x_rd ^ (4 * st))) * 4));
#pragma unroll
        for (int j = 0; j < VEC; ++j) {
          const F bv = __builtin_bit_cast(F, Num::bvals(DecW<VEC>::get(ch.w[st], j), magic));
          acc[j] = Mfma<DT>::m16(xa, bv, i == 0 ? f32x4{0.f, 0.f, 0.f, 0.f} : acc[j]);
        }
        xs = Mfma<DT>::m16(xa, ones, i == 0 ? f32x4{0.f, 0.f, 0.f, 0.f} : xs);
      }
      // QS * sum x (q - z) = acc - (OFF + QS z) xs, one fma per accumulator
      // (OFF + QS z is exact for the integer zero points of the format);
      // tot accumulates s times it
      float zc[VEC], sc[VEC];
#pragma unroll
      for (int j = 0; j < VEC; ++j) {
        zc[j] = __builtin_fmaf(Num::QS, ch.z[p].get(j), Num::OFF);
        sc[j] = ch.s[p].get(j);
      }
#pragma unroll
      for (int r = 0; r < R; ++r)
#pragma unroll
        for (int j = 0; j < VEC; ++j) {
          const float u = __builtin_fmaf(-zc[j], xs[r], acc[j][r]);
          tot[j][r] = __builtin_fmaf(sc[j], u, tot[j][r]);
        }
    }
    __builtin_amdgcn_wave_barrier();  // slots are rewritten by the next chunk
  };

  // Ring of D chunks: chunk t + D is loaded as soon as chunk t is consumed.
  // Loads are unconditional (a chunk past the run reads out of range: zeros,
  // no traffic), so the compiler's waits stay exact; computing a chunk past
  // the run is skipped with a scalar branch that contains no load.
  Chunk ring[D];
#pragma unroll
  for (int d = 0; d < D; ++d) load_chunk(ring[d], wb + d * C);
  for (int sb = wb; sb < we; sb += D * C) {
#pragma unroll
    for (int d = 0; d < D; ++d) {
      if (d == 0 || sb + d * C < we) compute_chunk(ring[d]);
      load_chunk(ring[d], sb + (d + D) * C);
    }
  }

  // cross-wave reduction in wave order; !ONE: each wave's partial tile goes
  // to its own activation area, which no other wave touches and which the
  // wave itself no longer reads
  float* const rbase = ONE ? red : reinterpret_cast<float*>(xl);
  const int rstride = ONE ? M * TN : MX * C4 * 4;
  if (ONE ? kb == 0 : true) {
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const int m = ONE ? 0 : kb * 4 + r;
      if (m < M) {
#pragma unroll
        for (int j = 0; j < VEC; ++j) rbase[wv * rstride + m * TN + VEC * c + j] = tot[j][r];
      }
    }
  }
  __syncthreads();
  const int total = M * TN;
  for (int idx = tid; idx < total; idx += kDecThreads) {
    const int m = idx / TN;
    const int nl = idx - m * TN;
    const int n = n0 + nl;
    if (n >= N) continue;
    float s = rbase[m * TN + nl];
#pragma unroll
    for (int w = 1; w < kDecWaves; ++w) s += rbase[w * rstride + m * TN + nl];
    a.y[(int64_t)m * a.ldy + n] = float_to_act_bits<DT>(s * (1.0f / Num::QS));
  }
}

// ------------------------------- dec_kernel_one (one workgroup per CU tile)
//
// One workgroup of 16 waves per CU-sized unit of work: a column tile of about
// 128 KB of packed weights (over the whole K, or one K part of a long K), so
// that the seven linears of an M = 1 decoder block become about 230 equal
// workgroups, at most one per CU.  Every
// wave issues all loads of its run (a round of NL 128-bit weight loads per
// lane, plus one load each for the round's activations, scales and zeros)
// before it waits for any of them; for K <= 8192 a round is the whole run, so
// a workgroup exposes one memory latency.
//
// Column tiles (four columns per lane, 128-bit weight loads, rows read in
// full 128-byte lines or longer):
//   T128 (K <= 2048): lane l = (quad l % 32, row l / 32); a load step covers
//        2 qweight rows (16 k) x 512 bytes.  In the 16x16x32 MFMA the four
//        k slices are (row, column half) = (0,0) (0,1) (1,0) (1,1); the A
//        operand of rows m < 8 is zero in the odd slices and that of rows
//        m >= 8 in the even slices, so row 0 of the result holds columns
//        0..63 and row 8 columns 64..127.
//   T64  (K <= 4096): lane l = (quad l % 16, row l / 16); 4 rows (32 k) x 256
//        bytes per step; all A rows equal, row 0 holds the 64 columns.
//   T32  (longer K): lane l = (quad l % 8, row l / 8); 8 rows (64 k) x 128
//        bytes per step.  Lanes l and l + 8 share a k slice but carry
//        different rows, so row 0 / columns 0..7 of the result sums the even
//        rows and row 8 / columns 8..15 the odd rows; the two halves are
//        corrected with their own activation sums and added in the final
//        reduction.
// Activations (permuted to the nibble order), scales and zeros are staged in
// a per-wave LDS area that only the wave itself reads (no barrier).
//
// Up to four activation rows (MR = 4, 2 <= M <= 4): A-operand row r carries
// activation row r % 4 (T128 and T32 keep their two halves, rows 0..3 and
// 8..11; rows 4..7 and 12..15 repeat them and are ignored), rows past M are
// staged as zeros, and the accumulator elements 0..3 of the owner lanes hold
// the rows 0..3 of their columns, each corrected with its own activation sum.
constexpr int kOneWaves = 16;
constexpr int kOneThreads = 64 * kOneWaves;
// per wave: activations (1 KB per row; 512 B per row for MR = 16, which has
// the 64-column tiling only), scales 1 KB, zeros 1 KB; then the reduction
// area, MR x 128 floats per wave (MR = 8 / 16: each wave's partials go to
// its own activation area, which only it has used: 8 x 128 floats in 8 KB,
// 16 x 64 floats in 16 x 512 B)
constexpr int one_xrow(int mr) { return mr == 16 ? 512 : 1024; }
constexpr int one_wave_lds(int mr) { return mr * one_xrow(mr) + 2048; }
constexpr int one_red_offset(int mr) { return kOneWaves * one_wave_lds(mr); }
constexpr int one_lds(int mr) {
  return one_red_offset(mr) + (mr >= 8 ? 0 : kOneWaves * mr * 128 * (int)sizeof(float));
}

constexpr int kMaxKSplit = 8;  // K parts of one M == 1 column tile
constexpr int kMaxRowSlices = 8;  // 16-row slices of one problem (M <= 128)

// K-split tile (M == 1): wave 0 sums the per-wave partials of each of the
// tile's columns (one or two per lane, the fixed wave order of the unsplit
// reduction), then the parts of a column combine pairwise up a fixed binary
// tree (parts 2i and 2i+1 first, then those pairs, ...).  Each tree node is a
// 64-bit word, zero when free: a part arriving at a node swaps in
// (1 << 32 | bits of its value) with one compare-and-swap; if the word was
// zero it leaves, otherwise it received its sibling's value, adds it, frees
// the word and climbs.  IEEE addition is commutative (a + b and b + a give the
// same bits), so whichever sibling arrives second computes the same sum: the
// result is a function of the inputs only, and the last part's critical path
// is one atomic round trip per tree level, with no cache flush and no
// partial-sum buffer (the value travels in the atomic).
// red: the per-wave partial tiles of the cross-wave reduction, wave w's
// column nl at red[w * RSTR + nl]
template <int DT, int TW, int RSTR>
__device__ __forceinline__ void dec_split_finish(const DecArgs& a, const float* red, int ct, int kp, int ks, int n0,
                                                 int lane) {
  typedef DecNum<DT> Num;
  static_assert(TW % 64 == 0, "split tiles: whole lanes per column");
  constexpr int C = TW / 64;
  unsigned long long* words = a.pair + (int64_t)ct * (ks - 1) * TW;
#pragma unroll
  for (int c = 0; c < C; ++c) {
    const int nl = c * 64 + lane;
    float pv[kOneWaves];
#pragma unroll
    for (int w = 0; w < kOneWaves; ++w) pv[w] = red[w * RSTR + nl];
    float v = 0.0f;
#pragma unroll
    for (int w = 0; w < kOneWaves; ++w) v += pv[w];
    v *= 1.0f / Num::QS;
    bool live = true;
    int base = 0;
    for (int width = ks >> 1, node = kp >> 1; width >= 1; base += width, width >>= 1, node >>= 1) {
      if (live) {
        unsigned long long* wd = words + (int64_t)(base + node) * TW + nl;
        unsigned long long seen = 0ull;
        const unsigned long long mine = (1ull << 32) | (unsigned long long)__builtin_bit_cast(uint32_t, v);
        if (__hip_atomic_compare_exchange_strong(wd, &seen, mine, __ATOMIC_RELAXED, __ATOMIC_RELAXED,
                                                 __HIP_MEMORY_SCOPE_AGENT)) {
          live = false;  // first of the pair: the sibling finishes
        } else {
          v += __builtin_bit_cast(float, (uint32_t)seen);
          __hip_atomic_store(wd, 0ull, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
      }
    }
    if (live && n0 + nl < a.N) {
      if (v != v) v = __builtin_bit_cast(float, 0x7FC00000u);  // one NaN pattern whatever the order
      a.y[n0 + nl] = float_to_act_bits<DT>(v);
    }
  }
}

// WV: waves of the workgroup.  sl0: the 16-row slice of the problem this
// workgroup computes (the eight-wave sixteen-row kernel; otherwise 0)
template <int DT, int TW, int GSI, int NL, int D, int MR, int WV = kOneWaves>
__device__ __forceinline__ void dec_tile_one(const DecArgs& a, int tile, uint8_t* lds, int sl0 = 0) {
  typedef typename Act<DT>::frag F;
  typedef DecNum<DT> Num;
  constexpr int RPS = TW == 128 ? 2 : TW == 64 ? 4 : 8;  // qweight rows per load step
  constexpr int SK = 8 * RPS;                            // k per load step
  constexpr int SLOTS = RPS < 4 ? 4 : RPS;               // LDS activation slots per step
  constexpr int QPR = TW / 4;                            // lanes per qweight row
  constexpr int GS = GSI < NL ? GSI : NL;                // correction interval (steps)
  constexpr int NP = NL / GS;                            // correction points = staged groups
  constexpr int LPG = TW / 8;                            // lanes per staged group row (16 B)
  constexpr int XE = NL * RPS;                           // activation entries (8 k) per round and row
  constexpr int XLD = (MR * XE + 63) / 64;               // activation loads per round and lane
  constexpr int WLDS = one_wave_lds(MR);
  static_assert(MR == 1 || MR == 4 || MR == 8 || MR == 16, "activation rows");
  static_assert(MR != 16 || TW == 64, "sixteen rows: 64 columns (all A rows distinct)");
  static_assert(MR == 1 || D == 1, "several rows: single-round tilings only");
  static_assert(NL * SLOTS * 16 <= one_xrow(MR), "per-row staging");
  constexpr int RE = MR < 4 ? MR : 4;  // result rows per lane (accumulator elements used)
  static_assert(XE <= 64 && NP * LPG <= 64 && NL * SLOTS * 16 <= 1024, "per-wave staging area");
  static_assert(GSI >= 1 && (NL % GS) == 0, "correction interval");

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wv = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int lq = lane % QPR, lr = lane / QPR;  // load quad and row within a step
  // A-operand slot within a step (T128: slots 2 and 3 stay zero) and the
  // activation row of this lane's A-operand row
  int a_slot = lr;
  if constexpr (TW == 128) a_slot = (((lane & 15) >> 3) == ((lane >> 4) & 1)) ? (lane >> 5) : 2;
  const int a_row = lane & (MR - 1);
  // activation row of accumulator element e of this lane (A rows 4 (lane / 16) + e)
  const int r_base = MR == 16 ? 4 * (lane >> 4) : MR == 8 ? 4 * ((lane >> 4) & 1) : 0;
  // result owners: output quad oq (columns 4 oq .. 4 oq + 3) and part
  bool owner;
  int oq, part = 0;
  if constexpr (TW == 128) {
    owner = MR == 8 || lane < 16 || (lane >= 32 && lane < 48);
    oq = lane < 32 ? (lane & 15) : 16 + (lane & 15);
  } else if constexpr (TW == 64) {
    owner = MR == 16 ? true : MR == 8 ? lane < 32 : lane < 16;
    oq = lane & 15;
  } else if constexpr (MR == 8) {
    // lane groups 0 / 1: even rows (columns 0..7 of the result), rows 0..3 /
    // 4..7; groups 2 / 3: odd rows (columns 8..15)
    owner = ((lane & 15) < 8) == (lane < 32);
    oq = lane & 7;
    part = lane >= 32 ? 1 : 0;
  } else {
    owner = lane < 8 || (lane >= 40 && lane < 48);
    oq = lane & 7;
    part = lane >= 40 ? 1 : 0;
  }
  const int N = a.N, K = a.K;
  // K split (64-column tiles only when M > 1): column tile ct, part kp of ks,
  // steps [s0, s0 + S); ks is a power of two, so shifts replace the integer
  // divisions (the prologue before the first load is on every workgroup's
  // critical path: 7-launch M = 1 block 29.8 -> 28.9 us)
  const int ks = MR == 1 || TW == 64 ? a.ksplit : 1;
  const int ks_log = __builtin_ctz((unsigned)ks);
  const int ct = tile >> ks_log;
  const int kp = tile - (ct << ks_log);
  const int n0 = ct * TW;
  const int S = (int)((unsigned)K / (unsigned)SK) >> ks_log;
  const int s0 = kp * S;
  const int per_wave = ((S + WV - 1) / WV + NL - 1) / NL * NL;
  const int wb = s0 + min(S, wv * per_wave);
  const int we = s0 + min(S, min(S, wv * per_wave) + per_wave);
  // Row slices (sixteen-row kernel, problems of more than 16 rows): the
  // workgroup computes its column tile (or K part) for rows [16 sl0,
  // 16 sl0 + M) of the problem.
  const int M = MR == 1 ? 1 : MR == 16 ? min(16, a.M - 16 * sl0) : a.M;

  const __amdgpu_buffer_rsrc_t rq =
      __builtin_amdgcn_make_buffer_rsrc((void*)a.qw, (short)0, (int)a.qw_bytes, kDecBufFlags);
  const __amdgpu_buffer_rsrc_t rs =
      __builtin_amdgcn_make_buffer_rsrc((void*)a.sc, (short)0, (int)a.sz_bytes, kDecBufFlags);
  const __amdgpu_buffer_rsrc_t rz =
      __builtin_amdgcn_make_buffer_rsrc((void*)a.ze, (short)0, (int)a.sz_bytes, kDecBufFlags);
  // activations of the slice's rows (one slice: the problem's range)
  const bool sliced = MR == 16 && a.slices > 1;
  const __amdgpu_buffer_rsrc_t rx = __builtin_amdgcn_make_buffer_rsrc(
      (void*)(sliced ? a.x + (int64_t)16 * sl0 * a.sxm : a.x), (short)0,
      sliced ? (int)(((int64_t)(M - 1) * a.sxm + K) * 2) : (int)a.x_bytes, kDecBufFlags);

  const uint32_t step_bytes = (uint32_t)RPS * 4u * (uint32_t)N;
  const uint32_t w_lane = ((uint32_t)lr * (uint32_t)N + (uint32_t)(n0 + 4 * lq)) * 4u;
  // activation entry f = 64 j + lane of a round: row f / XE, entry f % XE
  // (k8 row sb * RPS + f % XE); entries of rows past M read zeros
  uint32_t x_lane[XLD];
#pragma unroll
  for (int j = 0; j < XLD; ++j) {
    const int f = 64 * j + lane, m = f / XE, e = f % XE;
    x_lane[j] = (f < MR * XE && m < M) ? ((uint32_t)m * (uint32_t)a.sxm + (uint32_t)e * 8u) * 2u : kDecOOB;
  }
  const uint32_t sz_oob = lane < NP * LPG ? 0u : kDecOOB;
  const uint32_t sz_lane = (uint32_t)(lane / LPG) * (uint32_t)N * 2u + (uint32_t)(n0 * 2 + (lane % LPG) * 16);
  uint8_t* x_lds = lds + wv * WLDS;
  // Activation staging: row m holds NL * SLOTS 16-byte chunks, chunk c (step
  // c / SLOTS, k slot c % SLOTS) stored at position c ^ (m % MR) of the row.
  // An A-fragment read serves 16 lanes with the same chunk of up to 16
  // different rows; rows are NL * SLOTS * 16 bytes apart (a multiple of the
  // 256-byte bank line), so without the XOR they would all hit the same four
  // banks (a 16-way conflict at sixteen rows); with it they cover distinct
  // bank quads.
  auto xpos = [&](int m, int c) { return (m * (NL * SLOTS) + (c ^ (m & (MR - 1)))) * 16; };
  uint8_t* s_lds = x_lds + MR * one_xrow(MR);
  uint8_t* z_lds = s_lds + 1024;
  const uint32_t magic = dec_magic_vgpr<DT>();
  const F ones = __builtin_bit_cast(F, u32x4{Num::ONES, Num::ONES, Num::ONES, Num::ONES});
  if constexpr (TW == 128) {
    // the zero A slots (2 and 3 of every step and row) are never rewritten
#pragma unroll
    for (int f = lane; f < 2 * NL * MR; f += 64) {
      const int m = f / (2 * NL), e = f % (2 * NL);
      *reinterpret_cast<u32x4*>(x_lds + xpos(m, (e >> 1) * SLOTS + 2 + (e & 1))) = u32x4{0u, 0u, 0u, 0u};
    }
  }

  struct Round {
    u32x4 w[NL];
    u32x4 x[XLD], s, z;
  };
  // Issue order = order of use: activations, scales, zeros, weights.
  auto load_round = [&](Round& r, int sb) {
    const uint32_t oob = sb < we ? 0u : kDecOOB;  // scalar
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int j = 0; j < XLD; ++j)
      r.x[j] = __builtin_amdgcn_raw_buffer_load_b128(rx, (x_lane[j] + (uint32_t)sb * RPS * 16u) | oob, 0, 0);
    const uint32_t g0 = (uint32_t)((sb * SK) >> a.gshift);
    const uint32_t so = (g0 * (uint32_t)N * 2u + sz_lane) | sz_oob | oob;
    r.s = __builtin_amdgcn_raw_buffer_load_b128(rs, so, 0, kDecWeightAux);
    r.z = __builtin_amdgcn_raw_buffer_load_b128(rz, so, 0, kDecWeightAux);
    __builtin_amdgcn_sched_barrier(0);
    const uint32_t vo = ((uint32_t)sb * step_bytes + w_lane) | oob;
#pragma unroll
    for (int i = 0; i < NL; ++i)
      r.w[i] = __builtin_amdgcn_raw_buffer_load_b128(rq, vo + (uint32_t)i * step_bytes, 0, kDecWeightAux);
    __builtin_amdgcn_sched_barrier(0);
  };

  f32x4 acc[4];
  f32x4 xs;
  float tot[4][RE];

  // stage the round's activations (permuted), scales and zeros
  auto stage_round = [&](const Round& r) {
#pragma unroll
    for (int j = 0; j < XLD; ++j) {
      const int f = 64 * j + lane, m = f / XE, e = f % XE;
      if (f < MR * XE)
        *reinterpret_cast<u32x4*>(x_lds + xpos(m, (e / RPS) * SLOTS + e % RPS)) = dec_perm_x(r.x[j]);
    }
    *reinterpret_cast<u32x4*>(s_lds + lane * 16) = r.s;
    *reinterpret_cast<u32x4*>(z_lds + lane * 16) = r.z;
    __builtin_amdgcn_wave_barrier();
  };
  auto compute_round = [&](const Round& r, int sb) {
#pragma unroll
    for (int p = 0; p < NP; ++p) {
#pragma unroll
      for (int i = 0; i < GS; ++i) {
        const int st = p * GS + i;
        const F xa = __builtin_bit_cast(
            F, *reinterpret_cast<const u32x4*>(x_lds + xpos(a_row, st * SLOTS + a_slot)));
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const F b = __builtin_bit_cast(F, Num::bvals(r.w[st][j], magic));
          acc[j] = Mfma<DT>::m16(xa, b, i == 0 ? f32x4{0.f, 0.f, 0.f, 0.f} : acc[j]);
        }
        xs = Mfma<DT>::m16(xa, ones, i == 0 ? f32x4{0.f, 0.f, 0.f, 0.f} : xs);
      }
      // staged group row of this point (the first staged row is the group of sb)
      const int gp = ((sb + p * GS) * SK >> a.gshift) - ((sb * SK) >> a.gshift);
      const u32x2 sv = *reinterpret_cast<const u32x2*>(s_lds + gp * TW * 2 + oq * 8);
      const u32x2 zv = *reinterpret_cast<const u32x2*>(z_lds + gp * TW * 2 + oq * 8);
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const float sj = half_bits_to_float((uint16_t)(sv[j >> 1] >> (16 * (j & 1))));
        const float zj = half_bits_to_float((uint16_t)(zv[j >> 1] >> (16 * (j & 1))));
#pragma unroll
        for (int e = 0; e < RE; ++e) {
          const float u = __builtin_fmaf(-zj, Num::QS * xs[e], acc[j][e] - Num::OFF * xs[e]);
          tot[j][e] = __builtin_fmaf(sj, u, tot[j][e]);
        }
      }
    }
    __builtin_amdgcn_wave_barrier();  // the next round rewrites the staging area
  };
  auto clear_tot = [&]() {
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
      for (int e = 0; e < RE; ++e) tot[j][e] = 0.f;
  };

  // cross-wave (T32: and even/odd row) reduction in a fixed order; partials
  // of wave w, row m at red + w * RSTR + m * 128
  // (MR = 16: rows 64 floats apart, the tile is 64 columns)
  constexpr int RSTR = MR >= 8 ? WLDS / 4 : MR * 128;  // floats
  constexpr int RROW = MR == 16 ? 64 : 128;
  float* red = reinterpret_cast<float*>(lds + (MR >= 8 ? 0 : one_red_offset(MR)));

  // Reduce the workgroup's partials and store them (or, K split, publish
  // them; the last part to arrive stores the sum).  Slice sl0 has its own
  // rows of y, arrival counters and partial tiles.
  const int sl = sl0;
  auto finish = [&]() {
    uint16_t* const y = a.y + (int64_t)(16 * sl) * a.ldy;
    if (owner) {
      // the four columns of an output quad as one 16-byte store per row
#pragma unroll
      for (int e = 0; e < RE; ++e)
        *reinterpret_cast<f32x4*>(&red[wv * RSTR + (r_base + e) * RROW + part * 32 + 4 * oq]) =
            f32x4{tot[0][e], tot[1][e], tot[2][e], tot[3][e]};
    }
    __syncthreads();
    // Eight-wave sixteen-row kernel: each thread reduces two adjacent columns
    // of one row (64-bit LDS reads; the same adds in the same order as one
    // column per thread), so the tail is one round of reads for 512 threads.
    constexpr bool PAIR = MR * TW == 2 * WV * 64;
    if constexpr (PAIR) {
      const int el = 2 * tid, m = el / TW, nl = el - m * TW;
      float2 pv[WV];
#pragma unroll
      for (int w = 0; w < WV; ++w) pv[w] = *reinterpret_cast<const float2*>(&red[w * RSTR + m * RROW + nl]);
      __builtin_amdgcn_sched_barrier(0);
      float vx = 0.0f, vy = 0.0f;
#pragma unroll
      for (int w = 0; w < WV; ++w) vx += pv[w].x, vy += pv[w].y;
      const int n = n0 + nl;  // N % 8 == 0 on this kernel: n and n + 1 are both inside or both past N
      if (ks > 1) {
        // K split: publish the pair (one 64-bit device-coherent store), count
        // the part's arrival; the last part sums every part in part order
        // (the pair moves as a 64-bit buffer access with the sc1 policy, the
        // policy of agent-scope atomic loads and stores, ordered against the
        // arrival counter by the waits and barriers below)
        constexpr int E = MR * TW;
        unsigned* const cnt = a.cnt + (int64_t)sl * (a.col_tiles >> ks_log);
        float* const tiles = a.part + (int64_t)sl * a.col_tiles * E + (int64_t)ct * ks * E;
        const __amdgpu_buffer_rsrc_t rp =
            __builtin_amdgcn_make_buffer_rsrc((void*)tiles, (short)0, ks * E * (int)sizeof(float), kDecBufFlags);
        const u32x2 mine = u32x2{__builtin_bit_cast(uint32_t, vx), __builtin_bit_cast(uint32_t, vy)};
        __builtin_amdgcn_raw_buffer_store_b64(mine, rp, (uint32_t)(kp * E + el) * 4u, 0, kDecCoherentAux);
        __builtin_amdgcn_s_waitcnt(0);
        __syncthreads();  // every partial of this part has completed; red is no longer read
        unsigned* const arrived = reinterpret_cast<unsigned*>(lds);
        if (tid == 0) *arrived = __hip_atomic_fetch_add(cnt + ct, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        __syncthreads();
        if (*arrived != (unsigned)(ks - 1)) return;
        if (tid == 0) __hip_atomic_store(cnt + ct, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        u32x2 other[kMaxKSplit];
#pragma unroll
        for (int q = 0; q < kMaxKSplit; ++q)
          other[q] = (q < ks && q != kp)
                         ? __builtin_amdgcn_raw_buffer_load_b64(rp, (uint32_t)(q * E + el) * 4u, 0, kDecCoherentAux)
                         : mine;
        vx = 0.0f, vy = 0.0f;
#pragma unroll
        for (int q = 0; q < kMaxKSplit; ++q)
          if (q < ks) {
            // (the whole vector is bit-cast: a bit cast of one element of an
            // ext_vector_type value reads the vector's first element)
            const float2 f = __builtin_bit_cast(float2, other[q]);
            vx += f.x;
            vy += f.y;
          }
      }
      if (m < M && n < N) {
        y[(int64_t)m * a.ldy + n] = float_to_act_bits<DT>(vx * (1.0f / Num::QS));
        y[(int64_t)m * a.ldy + n + 1] = float_to_act_bits<DT>(vy * (1.0f / Num::QS));
      }
      return;
    }
    if constexpr (MR == 1 && TW % 64 == 0) {
      if (ks > 1) {
        if (wv == 0) dec_split_finish<DT, TW, RSTR>(a, red, ct, kp, ks, n0, lane);
        return;
      }
    }
    if constexpr (MR > 1 && TW == 64) {
      if (ks > 1) {
        // Several rows, K split: each part publishes its MR x 64 partial tile
        // with device-coherent stores (sc1: written through to the point all
        // XCDs read from), waits until they have completed and bumps the
        // tile's counter; the part that arrives last reads the others' tiles
        // with device-coherent loads, sums all parts in part order (so the
        // result does not depend on which part is last) and writes y, then
        // leaves the counter at zero.  Thread tid < MR * TW owns element tid
        // of the tile.  Slice sl has its own counters and partial tiles.
        constexpr int E = MR * TW;
        constexpr int EPT = (E + WV * 64 - 1) / (WV * 64);  // tile elements per thread
        unsigned* const cnt = a.cnt + (int64_t)sl * (a.col_tiles >> ks_log);
        float* const tiles = a.part + (int64_t)sl * a.col_tiles * E + (int64_t)ct * ks * E;
        float v[EPT];
#pragma unroll
        for (int i = 0; i < EPT; ++i) {
          const int el = tid + i * WV * 64, m = el / TW, nl = el - m * TW;
          v[i] = 0.0f;
          if (el < E) {
            float pv[WV];
#pragma unroll
            for (int w = 0; w < WV; ++w) pv[w] = red[w * RSTR + m * RROW + nl];
#pragma unroll
            for (int w = 0; w < WV; ++w) v[i] += pv[w];
            __hip_atomic_store(tiles + kp * E + el, v[i], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
          }
        }
        __builtin_amdgcn_s_waitcnt(0);
        __syncthreads();  // every partial of this part has completed; red is no longer read
        unsigned* const arrived = reinterpret_cast<unsigned*>(lds);
        if (tid == 0) *arrived = __hip_atomic_fetch_add(cnt + ct, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        __syncthreads();
        if (*arrived == (unsigned)(ks - 1)) {
          if (tid == 0) __hip_atomic_store(cnt + ct, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
#pragma unroll
          for (int i = 0; i < EPT; ++i) {
            const int el = tid + i * WV * 64, m = el / TW, nl = el - m * TW;
            if (el < E) {
              float other[kMaxKSplit];
#pragma unroll
              for (int p = 0; p < kMaxKSplit; ++p)
                other[p] = (p < ks && p != kp)
                               ? __hip_atomic_load(tiles + p * E + el, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT)
                               : v[i];
              float sum = 0.0f;
#pragma unroll
              for (int p = 0; p < kMaxKSplit; ++p)
                if (p < ks) sum += other[p];
              const int n = n0 + nl;
              if (m < M && n < N) y[(int64_t)m * a.ldy + n] = float_to_act_bits<DT>(sum * (1.0f / Num::QS));
            }
          }
        }
        return;
      }
    }
    for (int el = tid; el < MR * TW; el += WV * 64) {
      const int m = el / TW, nl = el - m * TW;
      const int n = n0 + nl;
      if (m < M && n < N) {
        // every partial is read before the first add (one LDS latency instead
        // of one per few reads); the adds keep the wave order
        constexpr int NPART = TW == 32 ? 2 * WV : WV;
        float pv[NPART];
#pragma unroll
        for (int w = 0; w < WV; ++w) {
          const float* rw = red + w * RSTR + m * RROW;
          if constexpr (TW == 32) {
            pv[2 * w] = rw[nl];
            pv[2 * w + 1] = rw[32 + nl];
          } else {
            pv[w] = rw[nl];
          }
        }
        __builtin_amdgcn_sched_barrier(0);
        float v = 0.0f;
#pragma unroll
        for (int i = 0; i < NPART; ++i) v += pv[i];
        y[(int64_t)m * a.ldy + n] = float_to_act_bits<DT>(v * (1.0f / Num::QS));
      }
    }
  };

  if constexpr (D == 1) {
    // the host picks D == 1 only when a wave's run fits in one round
    clear_tot();
    if (wb < we) {
      Round r;
      load_round(r, wb);
      stage_round(r);
      compute_round(r, wb);
    }
    finish();
  } else {
    clear_tot();
    Round ra, rb;
    load_round(ra, wb);
    load_round(rb, wb + NL);
    for (int sb = wb; sb < we; sb += 2 * NL) {
      stage_round(ra);
      compute_round(ra, sb);
      load_round(ra, sb + 2 * NL);
      if (sb + NL < we) {
        stage_round(rb);
        compute_round(rb, sb + NL);
      }
      load_round(rb, sb + 3 * NL);
    }
    finish();
  }
}

template <int DT, int GC, int MR>
__global__ __launch_bounds__(kOneThreads) void dec_kernel_one(DecGroupedArgs g) {
  __shared__ __attribute__((aligned(16))) float dec_smem[one_lds(MR) / 4];
  const int t = blockIdx.x;
  int p = 0;
#pragma unroll
  for (int i = 1; i < W4_MAX_GROUPED; ++i)
    if (i < g.count && t >= g.wg_start[i]) p = i;
  const DecArgs& a = g.prob[p];
  const int tile = t - g.wg_start[p];
  uint8_t* lds = reinterpret_cast<uint8_t*>(dec_smem);
  // steps per group (GC = log2(group / 32), 4 meaning >= 512)
  constexpr int G128 = 2 << GC;
  constexpr int G64 = 1 << GC;
  constexpr int G32 = GC >= 1 ? (1 << (GC - 1)) : 1;  // the host uses T32 for groups >= 64 only
  if constexpr (MR == 1) {
    switch (a.cfg) {
      case kCfgT128: dec_tile_one<DT, 128, G128, 8, 1, 1>(a, tile, lds); break;
      case kCfgT64: dec_tile_one<DT, 64, G64, 8, 1, 1>(a, tile, lds); break;
      case kCfgT64Ring: dec_tile_one<DT, 64, G64, 4, 2, 1>(a, tile, lds); break;
      case kCfgT32: dec_tile_one<DT, 32, G32, 8, 1, 1>(a, tile, lds); break;
      default: dec_tile_one<DT, 32, G32, 4, 2, 1>(a, tile, lds); break;
    }
  } else if constexpr (MR == 4) {
    // the host gives four-row launches single-round tilings only
    switch (a.cfg) {
      case kCfgT128: dec_tile_one<DT, 128, G128, 8, 1, MR>(a, tile, lds); break;
      case kCfgT64: dec_tile_one<DT, 64, G64, 8, 1, MR>(a, tile, lds); break;
      default: dec_tile_one<DT, 32, G32, 8, 1, MR>(a, tile, lds); break;
    }
  } else if constexpr (MR == 8) {
    // single-round tilings only, as for four rows
    switch (a.cfg) {
      case kCfgT128: dec_tile_one<DT, 128, G128, 8, 1, MR>(a, tile, lds); break;
      case kCfgT64: dec_tile_one<DT, 64, G64, 8, 1, MR>(a, tile, lds); break;
      default: dec_tile_one<DT, 32, G32, 8, 1, MR>(a, tile, lds); break;
    }
  }
}

// Problems of more than 16 rows (17 <= M <= 128), one 16-row slice per
// workgroup: eight waves over 64-column tiles and K parts of at most 2048 (8
// waves x 8 steps of 32 k), 80 KB of LDS and at most 128 VGPRs, so that two
// workgroups share a CU and one's memory wait overlaps the other's
// arithmetic.  (The sixteen-wave kernel leaves half of its waves idle at
// K = 2048 and holds the whole LDS, one workgroup per CU: the grouped
// decoder block at M = 64 took 37.7 us on it.)
constexpr int kSliceWaves = 8;
template <int DT, int GC>
__global__ __launch_bounds__(64 * kSliceWaves) __attribute__((amdgpu_waves_per_eu(4))) void dec_kernel_slices(
    DecGroupedArgs g) {
  __shared__ __attribute__((aligned(16))) float dec_smem[kSliceWaves * one_wave_lds(16) / 4];
  const int t = blockIdx.x;
  int p = 0;
#pragma unroll
  for (int i = 1; i < W4_MAX_GROUPED; ++i)
    if (i < g.count && t >= g.wg_start[i]) p = i;
  const DecArgs& a = g.prob[p];
  const int tile = t - g.wg_start[p];
  constexpr int G64 = 1 << GC;
  // Workgroup order: blocks of 8 column tiles x all slices, slice-major
  // inside a block, so the slices of one column tile are dispatched within
  // 8 * slices consecutive workgroups, all to the same XCD (workgroups go to
  // the XCDs round-robin and 8 divides the block stride): their reads of the
  // tile's weights meet in that XCD's L2 at about the same time.  Column
  // tiles past the last whole block of 8 follow, slice-major.
  const int S = a.slices, T = a.col_tiles;
  const int full = T & ~7;
  int sl, ct;
  if (tile < full * S) {
    const int blk = tile / (8 * S), r = tile - blk * 8 * S;
    sl = r >> 3;
    ct = blk * 8 + (r & 7);
  } else {
    const int rem = T - full, r = tile - full * S;
    sl = r / rem;
    ct = full + (r - sl * rem);
  }
  dec_tile_one<DT, 64, G64, 8, 1, 16, kSliceWaves>(a, ct, reinterpret_cast<uint8_t*>(dec_smem), sl);
}

template <int DT, bool ONE, int GS, int MX>
__global__ __launch_bounds__(kDecThreads) void dec_kernel(DecGroupedArgs g) {
  extern __shared__ __attribute__((aligned(16))) float dec_smem[];
  const int t = blockIdx.x;
  int p = 0;
#pragma unroll
  for (int i = 1; i < W4_MAX_GROUPED; ++i)
    if (i < g.count && t >= g.wg_start[i]) p = i;
  const DecArgs& a = g.prob[p];
  const int tile = t - g.wg_start[p];
  // LDS, ONE: [activation slots: 8 waves x 64 x 16 B][reduction: 8 waves x 64 floats];
  // !ONE: [activation areas: 8 waves x MX x 4C x 16 B], reused for the reduction
  uint32_t* xl = reinterpret_cast<uint32_t*>(dec_smem);
  float* red = dec_smem + kDecWaves * 64 * 4;
  if constexpr (MX == 16) {  // problems of more rows in 16-row slices
    int st = tile;
    const DecArgs as = dec_row_slice(a, st);
    if (as.vec == 4)
      dec_tile<DT, 4, ONE, (GS < 4 ? GS : 4), MX>(as, st, red, xl);
    else if (as.vec == 2)
      dec_tile<DT, 2, ONE, GS, MX>(as, st, red, xl);
    else
      dec_tile<DT, 1, ONE, GS, MX>(as, st, red, xl);
  } else if (a.vec == 4)
    dec_tile<DT, 4, ONE, (GS < 4 ? GS : 4), MX>(a, tile, red, xl);
  else if (a.vec == 2)
    dec_tile<DT, 2, ONE, GS, MX>(a, tile, red, xl);
  else
    dec_tile<DT, 1, ONE, GS, MX>(a, tile, red, xl);
}

}  // namespace w4

// ------------------------------------------------------------------- host side
using namespace w4host;

namespace {

bool dec_fits_32bit(int64_t N, int64_t K) {
  return N > 0 && K > 0 && N < (1LL << 27) && K < (1LL << 30) && (K / 8) * N * 4 < (1LL << 31);
}

struct DecPlan {
  w4::DecGroupedArgs g;
  int wgs;
  int gs;         // group-size class of the chosen kernel
  int mx;         // dec_kernel, M > 1: activation rows staged per wave (4, 8 or 16)
  bool cu_tiles;  // M == 1 one-workgroup-per-CU kernel (dec_kernel_one)
  bool sliced;    // cu_tiles with problems of more than 16 rows (dec_kernel_slices)
  int threads;
  size_t lds;
  // K-split problems (M == 1): their pairing words, as 64-bit word offsets
  // into the workspace's counter area
  int64_t pair_words;
  int64_t pair_off[W4_MAX_GROUPED];
  // K-split problems (M > 1): arrival counters (32-bit word offsets into the
  // counter area) and partial tiles (float offsets into the scratch)
  int64_t cnt_words, part_floats;
  int64_t cnt_off[W4_MAX_GROUPED], part_off[W4_MAX_GROUPED];
};

// Several rows (2 <= M <= 64), one workgroup per CU: the 64-column tiles
// hold K <= 4096 in one round, so a longer K (down_proj, 8192) is cut into
// ks parts (a power of two, whole groups and 256-k rounds), each part a
// workgroup of 64 columns x K / ks, combined by the last part to arrive
// (dec_tile_one).  Against 32-column tiles over all of K (128-byte pieces
// of the qweight rows: the four- and eight-row tilings, and the generic
// kernel beyond eight rows), this reads 256-byte pieces with all loads of a
// wave in flight at once.  Returns 1 for K <= 4096, 0 when no such split
// exists.
// `deeper` halves the parts again that many times while they stay whole
// groups and rounds: a lone down_proj at M = 16 has only 32 column tiles.
//
// Every several-row kernel runs rounds of 8 steps (256 k) per wave: one round
// of the sixteen-wave kernels holds K <= 4096, one of the eight-wave kernel
// for problems of more than 16 rows K <= 2048 (`part`).
int sixteen_ksplit(int64_t K, int G, int deeper, int64_t part) {
  const int64_t round = 256;
  if (K <= part) return 1;
  auto ok = [&](int k) {
    return k <= w4::kMaxKSplit && K % k == 0 && (K / k) % round == 0 && (K / k) % G == 0;
  };
  int ks = 2;
  while (K / ks > part) ks *= 2;
  if (!ok(ks)) return 0;
  for (int d = 0; d < deeper && ok(2 * ks); ++d) ks *= 2;
  return ks;
}

// M == 1, one workgroup per CU: problems with K > 4096 are cut into ksplit
// K parts of at most 4096 (ksplit a power of two) on 64-column tiles, i.e.
// 256-byte pieces of the qweight rows, instead of one 32-column tile over all
// of K (128-byte pieces).  Reading the decoder block's down_proj (2048 x 8192)
// as two K = 4096 halves or four K = 2048 quarters took 7.5 us for the grouped
// q/gate/up/down launch against 8.5 us with 32-column tiles (down_proj alone
// 4.6 against 7.1 us); the 32-column tiles were the last to finish, about
// 1.3 us after the rest.  A part must hold whole groups and whole load
// rounds of the 64-column tiling (8 steps of 32 k): a wave's round is masked
// as a whole past the end of its run, so a round that crossed into the next
// part would add that part's first steps a second time.
// Each narrowing level (a launch with few workgroups: a lone linear) halves
// the parts again while they stay whole rounds and groups, so a lone down_proj
// runs 256 workgroups of 32 KB instead of 64 of 128 KB.
// The pairing words ((ks - 1) per column) live in the workspace's counter area.
int one_ksplit(int64_t K, int G, int level, int64_t N) {
  if (K <= 4096 || G > 4096) return 1;
  int ks = 2;
  while (K / ks > 4096) ks *= 2;
  auto ok = [&](int k) {
    return k <= w4::kMaxKSplit && K % k == 0 && (K / k) % 256 == 0 && (K / k) % G == 0 &&
           (N + 63) / 64 * 64 * (int64_t)(k - 1) * 8 <= W4_WORKSPACE_COUNTER_BYTES;
  };
  if (!ok(ks)) return 1;
  for (int l = 0; l < level && ok(2 * ks); ++l) ks *= 2;
  return ks;
}

// Launch table: a pure function of shapes, strides and pointer alignment.
// Returns false (nothing launched) when a problem needs the general kernels:
// group size < 32, mixed group-size classes, misaligned or non-dense
// activations, or offsets past 2 GiB.
bool dec_plan(const w4a16_problem* problems, const int64_t* sxm, const int64_t* ldy, int count, int64_t M,
              DecPlan& dp, const int64_t* mrows = nullptr, bool split16 = false) {
  dp = DecPlan{};
  if (count < 1 || count > W4_MAX_GROUPED || M < 1 || M > 16) return false;
  struct Item {
    int idx;
    int vec, cfg, tile_n;
    int64_t tiles, bytes_per_wg;  // tiles: column tiles x K parts
    int ks, slices;
  } items[W4_MAX_GROUPED];
  int gclass = -1;
  // every problem fits the one-workgroup-per-CU tilings (M <= 16; for M > 1
  // only the single-round ones: K <= 8192, and K <= 4096 for group 32; for
  // M > 8 only the 64-column one: K <= 4096)
  bool cu_tiles = M <= 16;
  // sixteen-row launches (9 <= M <= 16, and problems of more rows in 16-row
  // slices): the eight-wave kernel, K parts <= 2048
  const bool sliced = M > 8;
  const int64_t part_k = sliced ? 2048 : 4096;
  for (int i = 0; i < count; ++i) {
    const w4a16_problem& q = problems[i];
    if (!dec_fits_32bit(q.N, q.K) || q.group_size < 32 || !is_pow2(q.group_size)) return false;
    if (gclass >= 0 && ilog2(q.group_size) != ilog2(problems[0].group_size)) return false;
    gclass = 0;
    if (((uintptr_t)q.x % 16) != 0) return false;
    // rows of this problem: at most M, or with M == 16 up to kMaxRowSlices
    // slices of 16 rows
    const int64_t Mi = mrows != nullptr ? mrows[i] : M;
    if (Mi < 1 || (Mi > M && (M != 16 || Mi > 16 * w4::kMaxRowSlices))) return false;
    if (M > 1 && ((sxm[i] % 8) != 0 || sxm[i] < q.K || ((Mi - 1) * sxm[i] + q.K) * 2 >= (1LL << 31))) return false;
    if (ldy != nullptr && ldy[i] < q.N) return false;
    const uintptr_t qa = (uintptr_t)q.qweight, sa = (uintptr_t)q.scales, za = (uintptr_t)q.zeros;
    cu_tiles = cu_tiles && q.N % 8 == 0 && qa % 16 == 0 && sa % 16 == 0 && za % 16 == 0;
    const bool split_ok = split16 && sixteen_ksplit(q.K, q.group_size, 0, part_k) > 1;
    if (M > 1 && M <= 8)
      cu_tiles = cu_tiles && ((q.K <= 8192 && (q.group_size >= 64 || q.K <= 4096)) || split_ok);
    if (M > 8) cu_tiles = cu_tiles && (q.K <= part_k || split_ok);
  }
  const int G = problems[0].group_size;
  // M == 1 tile width: about 128 KB of packed weights per workgroup (128
  // columns up to K = 2048, 64 up to 4096 or for group 32, else 32); each
  // narrowing level halves it where a tiling exists (128 -> 64 -> 32, the 32
  // column tiling needs groups >= 64).  A launch narrows while the narrower
  // grid still fits one workgroup per CU, so a lone small linear spreads over
  // the chip instead of a few CUs; a decoder block's 7 linears stay at level 0.
  auto one_width = [&](int64_t K, int level) {
    int tn = (K <= 2048 && M <= 8) ? 128 : (K <= 4096 || G < 64) ? 64 : 32;  // 16 rows: 64 only
    for (int l = 0; l < level; ++l) {
      if (tn == 128)
        tn = 64;
      else if (tn == 64 && G >= 64 && K <= 8192 && M <= 8)  // sixteen rows: no 32-column tiling
        tn = 32;
    }
    return tn;
  };
  // K-split tiles (M == 1 only): 128 columns over parts of K / ksplit
  auto tiles_at = [&](const w4a16_problem& q, int level) -> int64_t {
    const int ks = M == 1 ? one_ksplit(q.K, G, level, q.N) : 1;
    if (ks > 1) return (q.N + 63) / 64 * ks;
    const int tn = one_width(q.K, level);
    return (q.N + tn - 1) / tn;
  };
  int level = 0;
  int deeper = 0;  // sixteen rows: extra halvings of the K parts
  if (cu_tiles) {
    const int cus = device_cu_count();
    while (level < 2) {
      int64_t next = 0;
      for (int i = 0; i < count; ++i) next += tiles_at(problems[i], level + 1);
      if (next > cus) break;
      ++level;
    }
    if (M > 1 && split16) {
      // split K deeper while the launch still fits one workgroup per CU
      auto tiles16 = [&](int d) {
        int64_t t = 0;
        for (int i = 0; i < count; ++i) {
          const w4a16_problem& q = problems[i];
          const int64_t Mi = mrows != nullptr ? mrows[i] : M;
          const int k = sixteen_ksplit(q.K, q.group_size, d, part_k);
          t += (k > 1 ? (q.N + 63) / 64 * k : tiles_at(q, level)) * ((Mi + M - 1) / M);
        }
        return t;
      };
      while (deeper < 2 && tiles16(deeper + 1) > tiles16(deeper) && tiles16(deeper + 1) <= cus) ++deeper;
      // up to eight rows, K <= 8192 (group >= 64) also fits the unsplit
      // 32-column tiling:
      // split only where the parts spread over more CUs (a lone long-K
      // product); a launch that is already full (the grouped decoder block)
      // ran 0.4 us slower with the split's tail at M = 4
      if (M <= 8 && deeper == 0) {
        bool needed = false;  // a problem no single-round tiling holds
        for (int i = 0; i < count; ++i)
          needed = needed || problems[i].K > 8192 || (problems[i].group_size < 64 && problems[i].K > 4096);
        split16 = needed;
      }
    }
  }
  for (int i = 0; i < count; ++i) {
    const w4a16_problem& q = problems[i];
    const uintptr_t qa = (uintptr_t)q.qweight, sa = (uintptr_t)q.scales, za = (uintptr_t)q.zeros;
    int vec = 1, cfg = 0, tn = 16, ks = 1;
    if (cu_tiles) {
      vec = 4;
      // (sixteen_ksplit returns 0 where no split exists: those problems stay
      // whole, on the single-round tilings)
      ks = M == 1 ? one_ksplit(q.K, G, level, q.N) : split16 ? std::max(1, sixteen_ksplit(q.K, G, deeper, part_k)) : 1;
      tn = ks > 1 ? 64 : one_width(q.K, level);
      cfg = tn == 128 ? w4::kCfgT128
          : tn == 64  ? (q.K / ks <= 4096 ? w4::kCfgT64 : w4::kCfgT64Ring)
                      : (q.K <= 8192 ? w4::kCfgT32 : w4::kCfgT32Ring);
    } else if (q.N % 4 == 0 && qa % 16 == 0 && sa % 8 == 0 && za % 8 == 0 && q.K <= 4096) {
      vec = 4, tn = 64;
    } else if (q.N % 2 == 0 && qa % 8 == 0 && sa % 4 == 0 && za % 4 == 0) {
      vec = 2, tn = 32;
    }
    const int64_t Mi = mrows != nullptr ? mrows[i] : M;
    const int slices = (int)((Mi + M - 1) / M);  // > 1 only for 16-row launches
    items[i] = Item{i, vec, cfg, tn, (q.N + tn - 1) / tn * ks, (int64_t)tn * (q.K / ks) / 2, ks, slices};
  }
  // Longest-running workgroups first: more bytes, then longer K (narrower
  // tiles with more correction points per byte).
  std::stable_sort(items, items + count, [&](const Item& l, const Item& r) {
    if (l.bytes_per_wg != r.bytes_per_wg) return l.bytes_per_wg > r.bytes_per_wg;
    return problems[l.idx].K > problems[r.idx].K;
  });
  int wgs = 0;
  for (int s = 0; s < count; ++s) {
    const Item& it = items[s];
    const w4a16_problem& q = problems[it.idx];
    w4::DecArgs& a = dp.g.prob[s];
    a.x = static_cast<const uint16_t*>(q.x);
    a.qw = reinterpret_cast<const uint32_t*>(q.qweight);
    a.sc = q.scales;
    a.ze = q.zeros;
    a.y = static_cast<uint16_t*>(q.y);
    a.sxm = M > 1 ? sxm[it.idx] : 0;
    a.ldy = ldy != nullptr ? ldy[it.idx] : q.N;
    a.qw_bytes = (uint32_t)((q.K / 8) * q.N * 4);
    a.sz_bytes = (uint32_t)((q.K / q.group_size) * q.N * 2);
    const int64_t Mi = mrows != nullptr ? mrows[it.idx] : M;
    a.x_bytes = (uint32_t)(((Mi - 1) * a.sxm + q.K) * 2);
    a.N = (int)q.N;
    a.K = (int)q.K;
    a.M = (int)Mi;
    a.gshift = ilog2(q.group_size);
    a.vec = it.vec;
    a.cfg = it.cfg;
    a.ksplit = it.ks;
    a.pair = nullptr;
    a.slices = it.slices;
    a.col_tiles = (int)it.tiles;
    a.cnt = nullptr;
    a.part = nullptr;
    if (it.ks > 1 && M > 1) {
      const int mr = M <= 4 ? 4 : M <= 8 ? 8 : 16;  // rows of the launch's kernel
      dp.cnt_off[s] = dp.cnt_words;
      dp.part_off[s] = dp.part_floats;
      dp.cnt_words += it.tiles / it.ks * it.slices;  // per slice: one counter per column tile
      dp.part_floats += it.tiles * it.slices * mr * 64;
    }
    if (it.ks > 1 && M == 1) {
      dp.pair_off[s] = dp.pair_words;
      dp.pair_words += (it.tiles / it.ks) * (it.ks - 1) * it.tile_n;
    }
    dp.g.wg_start[s] = wgs;
    if (it.tiles * it.slices > (1 << 24)) return false;
    wgs += (int)(it.tiles * it.slices);
  }
  for (int s = count; s <= W4_MAX_GROUPED; ++s) dp.g.wg_start[s] = wgs;
  dp.g.count = count;
  dp.wgs = wgs;
  dp.cu_tiles = cu_tiles;
  dp.sliced = cu_tiles && sliced;
  if (cu_tiles) {
    dp.gs = std::min(ilog2(G) - 5, 4);  // dec_kernel_one: log2(group / 32), 4 = ">= 512"
    dp.threads = sliced ? 64 * w4::kSliceWaves : w4::kOneThreads;
    dp.lds = 0;  // static in dec_kernel_one
  } else {
    dp.gs = (int)std::min(G / 32, 8);  // dec_kernel: steps per group, capped at 8
    dp.threads = w4::kDecThreads;
    // rows staged per wave: the smallest width that holds M rows, except that
    // launches with more workgroups than CUs stage 8 rows for M <= 4 as well
    // (measured: the 7-linear block in one launch at M = 2 / 4 takes 10.8 /
    // 10.9 us with 8 rows against 12.2 / 12.4 us with 4, while launches of at
    // most one workgroup per CU are 6 % slower with 8); the rows fed to the
    // MFMA, and so every output bit, do not depend on it
    dp.mx = (M <= 4 && wgs <= device_cu_count()) ? 4 : M <= 8 ? 8 : 16;
    bool narrow = false;  // a tile of vec < 4 has chunks of 8 steps (32 slices per row)
    for (int s = 0; s < count; ++s) narrow = narrow || dp.g.prob[s].vec < 4;
    // ONE: activation slots + reduction; M > 1: activation areas (at most
    // 64 KB), which also hold the per-wave partial tiles (M x 64 floats <= MX x 4C x 16 B)
    dp.lds = M == 1 ? (size_t)w4::kDecWaves * 64 * 16 + (size_t)w4::kDecWaves * 64 * sizeof(float)
                    : (size_t)w4::kDecWaves * dp.mx * (narrow ? 32 : 16) * 16;
  }
  return wgs > 0;
}

template <int DT, int MR>
void dec_launch_one_mr(const DecPlan& dp, hipStream_t st) {
  const dim3 grid((unsigned)dp.wgs), block(w4::kOneThreads);
  switch (dp.gs) {
    case 0: hipLaunchKernelGGL((w4::dec_kernel_one<DT, 0, MR>), grid, block, dp.lds, st, dp.g); break;
    case 1: hipLaunchKernelGGL((w4::dec_kernel_one<DT, 1, MR>), grid, block, dp.lds, st, dp.g); break;
    case 2: hipLaunchKernelGGL((w4::dec_kernel_one<DT, 2, MR>), grid, block, dp.lds, st, dp.g); break;
    case 3: hipLaunchKernelGGL((w4::dec_kernel_one<DT, 3, MR>), grid, block, dp.lds, st, dp.g); break;
    default: hipLaunchKernelGGL((w4::dec_kernel_one<DT, 4, MR>), grid, block, dp.lds, st, dp.g); break;
  }
}

template <int DT>
void dec_launch_slices(const DecPlan& dp, hipStream_t st) {
  const dim3 grid((unsigned)dp.wgs), block(64 * w4::kSliceWaves);
  switch (dp.gs) {
    case 0: hipLaunchKernelGGL((w4::dec_kernel_slices<DT, 0>), grid, block, 0, st, dp.g); break;
    case 1: hipLaunchKernelGGL((w4::dec_kernel_slices<DT, 1>), grid, block, 0, st, dp.g); break;
    case 2: hipLaunchKernelGGL((w4::dec_kernel_slices<DT, 2>), grid, block, 0, st, dp.g); break;
    case 3: hipLaunchKernelGGL((w4::dec_kernel_slices<DT, 3>), grid, block, 0, st, dp.g); break;
    default: hipLaunchKernelGGL((w4::dec_kernel_slices<DT, 4>), grid, block, 0, st, dp.g); break;
  }
}

template <int DT>
void dec_launch_one(const DecPlan& dp, int64_t M, hipStream_t st) {
  if (dp.sliced)
    dec_launch_slices<DT>(dp, st);
  else if (M == 1)
    dec_launch_one_mr<DT, 1>(dp, st);
  else if (M <= 4)
    dec_launch_one_mr<DT, 4>(dp, st);
  else
    dec_launch_one_mr<DT, 8>(dp, st);
}

template <int DT, bool ONE, int MX>
void dec_launch_generic(const DecPlan& dp, hipStream_t st) {
  const dim3 grid((unsigned)dp.wgs), block(w4::kDecThreads);
  switch (dp.gs) {
    case 1: hipLaunchKernelGGL((w4::dec_kernel<DT, ONE, 1, MX>), grid, block, dp.lds, st, dp.g); break;
    case 2: hipLaunchKernelGGL((w4::dec_kernel<DT, ONE, 2, MX>), grid, block, dp.lds, st, dp.g); break;
    case 4: hipLaunchKernelGGL((w4::dec_kernel<DT, ONE, 4, MX>), grid, block, dp.lds, st, dp.g); break;
    default: hipLaunchKernelGGL((w4::dec_kernel<DT, ONE, 8, MX>), grid, block, dp.lds, st, dp.g); break;
  }
}

template <int DT>
void dec_launch(const DecPlan& dp, int64_t M, hipStream_t st) {
  if (dp.cu_tiles)
    dec_launch_one<DT>(dp, M, st);
  else if (M == 1)
    dec_launch_generic<DT, true, 1>(dp, st);
  else if (dp.mx == 4)
    dec_launch_generic<DT, false, 4>(dp, st);
  else if (dp.mx == 8)
    dec_launch_generic<DT, false, 8>(dp, st);
  else
    dec_launch_generic<DT, false, 16>(dp, st);
}

}  // namespace

// The several-row K split is used when its counters fit the counter area: a
// function of the shapes only, so a call without the workspace it needs fails
// (W4_ERR_WORKSPACE) instead of taking another summation order.  Grouped
// launches take it too although they then need more than one workgroup per
// CU: the 7-linear block in one launch at M = 16 / 32 / 64 took 11.9 / 21.2 /
// 39.1 us on the one-workgroup-per-CU kernel against 13.6 / 23.6 / 44.1 us on
// the generic kernel (which it replaces for these launches).
bool split16_shape_ok(const DecPlan& dp) { return dp.cnt_words * 4 <= W4_WORKSPACE_COUNTER_BYTES; }

bool dec_plan_final(const w4a16_problem* problems, const int64_t* sxm, const int64_t* ldy, int count, int64_t M,
                    DecPlan& dp, const int64_t* mrows) {
  if (!dec_plan(problems, sxm, ldy, count, M, dp, mrows, true)) return false;
  if (dp.cnt_words > 0 && !split16_shape_ok(dp)) return dec_plan(problems, sxm, ldy, count, M, dp, mrows, false);
  return true;
}

// Factored decode launch (see the top of this file).  Returns
// W4_ERR_UNSUPPORTED, with nothing launched and no error message, when the
// problems need the general kernels.  sxm: activation row strides, ldy: output
// row strides (elements; null = dense); mrows: rows of each problem (null: M
// for all; each <= M, the launch's row count, which picks the kernel).
int w4_decode_launch(const w4a16_problem* problems, const int64_t* sxm, const int64_t* ldy, int count,
                     int x_dtype, int64_t M, unsigned* counters, void* scratch, size_t scratch_bytes,
                     hipStream_t st, const int64_t* mrows) {
  DecPlan dp;
  if (!dec_plan_final(problems, sxm, ldy, count, M, dp, mrows)) return W4_ERR_UNSUPPORTED;
  if (dp.cnt_words > 0) {
    const size_t need = (size_t)dp.part_floats * 4;
    if (counters == nullptr || scratch == nullptr || scratch_bytes < need)
      return fail(W4_ERR_WORKSPACE, "w4a16 decode: a workspace of %zu bytes is required",
                  (size_t)W4_WORKSPACE_COUNTER_BYTES + need);
    for (int s = 0; s < dp.g.count; ++s) {
      w4::DecArgs& a = dp.g.prob[s];
      if (a.ksplit > 1) {
        a.cnt = counters + dp.cnt_off[s];
        a.part = static_cast<float*>(scratch) + dp.part_off[s];
      }
    }
  }
  if (dp.pair_words > 0) {
    // K-split problems: pairing words in the workspace's counter area
    if (dp.pair_words * 8 > W4_WORKSPACE_COUNTER_BYTES) return W4_ERR_UNSUPPORTED;
    if (counters == nullptr)
      return fail(W4_ERR_WORKSPACE, "w4a16 decode: a workspace of %d bytes is required",
                  (int)W4_WORKSPACE_COUNTER_BYTES);
    for (int s = 0; s < dp.g.count; ++s) {
      w4::DecArgs& a = dp.g.prob[s];
      if (a.ksplit > 1) a.pair = reinterpret_cast<unsigned long long*>(counters) + dp.pair_off[s];
    }
  }
  if (x_dtype == W4_DTYPE_BF16)
    dec_launch<W4_DTYPE_BF16>(dp, M, st);
  else
    dec_launch<W4_DTYPE_FP16>(dp, M, st);
  return check_launch("w4a16 decode");
}

// Workspace bytes w4_decode_launch needs for these problems: the counter area
// (which holds the pairing words of K-split problems), or 0 when the decode
// kernels do not take them or split nothing.  Pointers are only used for
// their alignment, so callers without buffers may pass 256-byte-aligned
// stand-ins.
size_t w4_decode_workspace_bytes(const w4a16_problem* problems, const int64_t* sxm, int count, int64_t M,
                                 const int64_t* mrows) {
  DecPlan dp;
  if (!dec_plan_final(problems, sxm, nullptr, count, M, dp, mrows)) return 0;
  if (dp.cnt_words > 0) return W4_WORKSPACE_COUNTER_BYTES + (size_t)dp.part_floats * 4;
  if (dp.pair_words == 0 || dp.pair_words * 8 > W4_WORKSPACE_COUNTER_BYTES) return 0;
  return W4_WORKSPACE_COUNTER_BYTES;
}

// Workspace bytes of one product's decode launch (w4a16_gemm: M <= 16 as is,
// 17 <= M <= 64 as 16-row slices), for dense aligned operands (stand-ins).
size_t w4_decode_single_workspace_bytes(int64_t M, int64_t N, int64_t K, int G) {
  static char aligned_stand_in[256] __attribute__((aligned(256)));
  const w4a16_problem q{aligned_stand_in, reinterpret_cast<const int32_t*>(aligned_stand_in),
                        reinterpret_cast<const uint16_t*>(aligned_stand_in),
                        reinterpret_cast<const uint16_t*>(aligned_stand_in), aligned_stand_in, N, K, G, 0};
  const int64_t sx = K;
  if (M <= 16) return w4_decode_workspace_bytes(&q, &sx, 1, M, nullptr);
  if (M > 16 * w4::kMaxRowSlices) return 0;
  return w4_decode_workspace_bytes(&q, &sx, 1, 16, &M);
}
