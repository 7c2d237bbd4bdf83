// Group-wise asymmetric RTN int4 quantize/pack and the exact dequantize, for
// gfx950.  Semantics follow the reference's torch implementation
// (int4_triton/quantize.py:102-135) bit for bit; the kernel structure is this
// library's own: one wave per (group, 64-column strip), min/max by wave
// shuffles, nibble packing in registers and an LDS transpose so that every
// qweight row segment is written as one coalesced 256-byte store.
#include <hip/hip_runtime.h>

#include <climits>

#include "w4_common.hpp"

namespace w4 {

__device__ __forceinline__ float max_nan(float a, float b) { return (a > b || a != a) ? a : b; }
__device__ __forceinline__ float min_nan(float a, float b) { return (a < b || a != a) ? a : b; }
// torch.clamp keeps NaN (quantize.py:108-113); fminf/fmaxf would drop it.
__device__ __forceinline__ float clamp_nan(float x, float lo, float hi) {
  return (x != x) ? x : fminf(fmaxf(x, lo), hi);
}

// NaN-propagating maximum / minimum (v_maximum3_f32 / v_minimum3_f32 on
// gfx950): a NaN anywhere in a group reaches the reduced extremes, as with
// torch's amax / amin (quantize.py:108-109); no input canonicalization.
__device__ __forceinline__ float fmax_p(float a, float b) { return __builtin_elementwise_maximum(a, b); }
__device__ __forceinline__ float fmin_p(float a, float b) { return __builtin_elementwise_minimum(a, b); }

template <int CTRL>
__device__ __forceinline__ float dpp_mov(float v) {
  return __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), CTRL, 0xF, 0xF, true));
}

// Maximum and minimum over aligned groups of L lanes (L a power of two up to
// 64): DPP steps inside rows of 16 lanes (swap neighbours, swap pairs,
// half-row mirror, row mirror), lane shuffles across rows.
template <int L>
__device__ __forceinline__ void group_minmax(float& mx, float& mn) {
  if constexpr (L >= 2) {
    mx = fmax_p(mx, dpp_mov<0xB1>(mx));  // quad_perm [1,0,3,2]
    mn = fmin_p(mn, dpp_mov<0xB1>(mn));
  }
  if constexpr (L >= 4) {
    mx = fmax_p(mx, dpp_mov<0x4E>(mx));  // quad_perm [2,3,0,1]
    mn = fmin_p(mn, dpp_mov<0x4E>(mn));
  }
  if constexpr (L >= 8) {
    mx = fmax_p(mx, dpp_mov<0x141>(mx));  // row_half_mirror
    mn = fmin_p(mn, dpp_mov<0x141>(mn));
  }
  if constexpr (L >= 16) {
    mx = fmax_p(mx, dpp_mov<0x140>(mx));  // row_mirror
    mn = fmin_p(mn, dpp_mov<0x140>(mn));
  }
  if constexpr (L >= 32) {
    mx = fmax_p(mx, __shfl_xor(mx, 16, 64));
    mn = fmin_p(mn, __shfl_xor(mn, 16, 64));
  }
  if constexpr (L >= 64) {
    mx = fmax_p(mx, __shfl_xor(mx, 32, 64));
    mn = fmin_p(mn, __shfl_xor(mn, 32, 64));
  }
}

struct QStats {
  float scale;  // fp16-representable (or 0/inf/NaN in degenerate groups)
  float zero;
};

// Fast form of group_stats, bit-identical to it, plus rcp(scale).
//  - scale: for x = wmax - wmin in [2^-90, 2^126], y = x * fl(1/15) followed
//    by one fma correction with the exact residual fma(-y, 15, x) is the
//    correctly rounded x / 15 (checked for every float in that range by
//    tests/div15_exhaustive.c); elsewhere the IEEE division.
//  - zero: -wmin / scale <= 22.5 (scale >= x / 15 up to the fp16 rounding,
//    which for a subnormal scale >= 2^-24 is at most 2^-25), so with
//    v_rcp_f32 within 1 ulp t0 = fma(-wmin, rcp(scale), 0.5) is within 6e-6
//    of the reference's fl(fl(-wmin / scale) + 0.5) and the floors agree
//    unless fract(t0) is within 2^-15 of 0 or 1, where, and for a zero /
//    infinite / NaN scale, the IEEE division is used.
__device__ __forceinline__ QStats group_stats_fast(float rmax, float rmin, float* rcp) {
#pragma clang fp contract(off)
  const float wmax = max_nan(rmax, 0.0f);
  const float wmin = min_nan(rmin, 0.0f);
  const float x = wmax - wmin;
  float scale;
  if (x >= 0x1p-90f && x <= 0x1p126f) {
    constexpr float C15 = 1.0f / 15.0f;
    const float y = x * C15;
    scale = __builtin_fmaf(__builtin_fmaf(-y, 15.0f, x), C15, y);
  } else {
    scale = x / 15.0f;
  }
  if (scale == 0.0f) scale = 1.0f;
  scale = (float)(_Float16)scale;
  const float r = __builtin_amdgcn_rcpf(scale);
  const float t0 = __builtin_fmaf(-wmin, r, 0.5f);
  const float f0 = __builtin_amdgcn_fractf(t0);
  float zero;
  if (scale > 0.0f && scale < __builtin_inff() && f0 >= 0x1p-15f && f0 <= 1.0f - 0x1p-15f)
    zero = __builtin_amdgcn_fmed3f(floorf(t0), 0.0f, 15.0f);
  else
    zero = clamp_nan(floorf(-wmin / scale + 0.5f), 0.0f, 15.0f);
  *rcp = r;
  QStats st;
  st.scale = scale;
  st.zero = zero;
  return st;
}

// quantize.py:108-112, in the same fp32 op order (true IEEE division).
__device__ __forceinline__ QStats group_stats(float rmax, float rmin) {
#pragma clang fp contract(off)
  const float wmax = max_nan(rmax, 0.0f);
  const float wmin = min_nan(rmin, 0.0f);
  float scale = (wmax - wmin) / 15.0f;
  if (scale == 0.0f) scale = 1.0f;
  scale = (float)(_Float16)scale;
  const float zero = clamp_nan(floorf(-wmin / scale + 0.5f), 0.0f, 15.0f);
  QStats r;
  r.scale = scale;
  r.zero = zero;
  return r;
}

// quantize.py:113-116: q = clamp(floor(w/scale + 0.5) + zero, 0, 15) -> int32
// (NaN converts to INT32_MIN like the reference's CPU cast), packed with
// int32 wrap-around.
__device__ __forceinline__ uint32_t quantize_pack8(const float v[8], QStats st) {
#pragma clang fp contract(off)
  uint32_t word = 0;
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const float qf = clamp_nan(floorf(v[i] / st.scale + 0.5f) + st.zero, 0.0f, 15.0f);
    const uint32_t q = (qf != qf) ? 0x80000000u : (uint32_t)(int)qf;
    word += q << (4 * i);
  }
  return word;
}

// Fast form of quantize_pack8 for finite weights and a finite nonzero scale
// (group_stats' scale is then in [2^-24, 65504]).  t = w * rcp(scale) + 0.5 +
// zero in one fma (zero is an integer in [0, 15]): v_rcp_f32 is within 1 ulp,
// so while |w/scale| < 32, t lies within 8e-6 of the reference's
// fl(fl(w/scale) + 0.5) + zero and both floors agree unless t is within 2^-15
// of an integer; beyond that range both clamp to the same end (0 or 15).
// q = trunc(med3(t, 0, 15.5)) is clamp(floor(t), 0, 15).  Returns true in
// *near when some fract(t) is within 2^-15 of 0 or 1: the caller then repacks
// the word with quantize_pack8.  Otherwise the word is bit-identical to
// quantize_pack8's.
__device__ __forceinline__ uint32_t quantize_pack8_fast(const float v[8], QStats st, float rcp, bool* near) {
  const float c = 0.5f + st.zero;
  uint32_t word = 0;
  float lo = 1.0f, hi = 0.0f;
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const float t = __builtin_fmaf(v[i], rcp, c);
    const float f = __builtin_amdgcn_fractf(t);
    lo = fmin_p(lo, f);
    hi = fmax_p(hi, f);
    word |= (uint32_t)__builtin_amdgcn_fmed3f(t, 0.0f, 15.5f) << (4 * i);
  }
  *near = !(lo >= 0x1p-15f && hi <= 1.0f - 0x1p-15f);
  return word;
}

// The eight activation-dtype weights of one 16-byte row segment, as floats.
template <int DT>
__device__ __forceinline__ void unpack_row8(const u32x4 r, float v[8]) {
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    v[2 * j] = act_bits_to_float((uint16_t)(r[j] & 0xFFFFu), DT);
    v[2 * j + 1] = act_bits_to_float((uint16_t)(r[j] >> 16), DT);
  }
}

// Stored fp16 patterns.  A NaN zero point is written as 0xFE00, the x86
// "default NaN" that the reference's CPU path produces for -0/0 and for
// negated NaN inputs; a NaN scale (NaN weights) as 0x7E00.
__device__ __forceinline__ uint16_t scale_bits(float s) {
  return (s != s) ? (uint16_t)0x7E00 : __builtin_bit_cast(uint16_t, (_Float16)s);
}
__device__ __forceinline__ uint16_t zero_bits(float z) {
  return (z != z) ? (uint16_t)0xFE00 : __builtin_bit_cast(uint16_t, (_Float16)z);
}

template <int DT, bool VEC>
__device__ __forceinline__ void load8(const uint16_t* __restrict__ w, int64_t n, int64_t k,
                                      int64_t swn, int64_t swk, float v[8]) {
  if (VEC) {
    const u32x4 p = *reinterpret_cast<const u32x4*>(w + n * swn + k);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      v[2 * i] = act_bits_to_float((uint16_t)(p[i] & 0xFFFFu), DT);
      v[2 * i + 1] = act_bits_to_float((uint16_t)(p[i] >> 16), DT);
    }
  } else {
#pragma unroll
    for (int i = 0; i < 8; ++i) v[i] = act_bits_to_float(w[n * swn + (k + i) * swk], DT);
  }
}

constexpr int QROWS = 64;  // columns n per tile (= lanes, for the stores)
constexpr int QWAVES = 4;  // waves per workgroup (two-pass kernel)
constexpr int QSWAVES = 8;  // waves per workgroup (single-pass kernel)

// Waves sharing one (group, 64-column) tile: 64 rows split between up to eight
// waves, each taking whole iterations of 512 / G rows (a lone wave per tile
// runs one long dependent chain per SIMD and leaves most of the chip idle).
constexpr int quantize_waves_per_tile(int G) { return G / 8 < QSWAVES ? G / 8 : QSWAVES; }

// Single-pass kernel for G <= 512: lanes_per_row = G/8 lanes each own one
// packed word of a row; 64/lanes_per_row rows are processed per iteration.
// One weight of a quantize launch (w4_quantize_grouped puts several in one).
struct QuantArgs {
  const uint16_t* w;
  int32_t* qw;
  uint16_t* sc;
  uint16_t* ze;
  int64_t N, K, swn, swk;
  int64_t tiles_n, tiles_total;
};

constexpr int kQuantMaxGrouped = 8;
struct QuantGroupedArgs {
  QuantArgs prob[kQuantMaxGrouped];
  int wg_start[kQuantMaxGrouped + 1];
  int count;
};

// The tiles of workgroup `blk` of one weight (see quantize_small_group_kernel).
template <int DT, int G, bool VEC>
__device__ __forceinline__ void quantize_small_group_tiles(const QuantArgs& qa, int blk) {
  const uint16_t* __restrict__ w = qa.w;
  int32_t* __restrict__ qw = qa.qw;
  uint16_t* __restrict__ sc = qa.sc;
  uint16_t* __restrict__ ze = qa.ze;
  const int64_t N = qa.N, K = qa.K, swn = qa.swn, swk = qa.swk, tiles_n = qa.tiles_n, tiles_total = qa.tiles_total;
  constexpr int L = G / 8;            // lanes per row (1..64)
  constexpr int RPI = 64 / L;         // rows per iteration
  constexpr int WPT = quantize_waves_per_tile(G);
  constexpr int TPB = QSWAVES / WPT;  // tiles per workgroup
  constexpr int RW = QROWS / WPT;     // rows per wave
  static_assert(RW % RPI == 0 && L % WPT == 0, "wave split of a tile");
  __shared__ uint32_t tile[TPB][L][QROWS + 1];
  __shared__ uint16_t st_s[TPB][QROWS];
  __shared__ uint16_t st_z[TPB][QROWS];

  const int lane = threadIdx.x & 63;
  const int wv = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // wave-uniform: tile math stays scalar
  const int ts = wv / WPT, sub = wv % WPT;  // tile slot, row slice of this wave
  // the host keeps tile counts below 2^31, so the tile index math is 32-bit
  const int t = blk * TPB + ts;
  const bool active = t < (int)tiles_total;
  const int g = active ? t / (int)tiles_n : 0;
  const int64_t n0 = active ? (int64_t)(t - g * (int)tiles_n) * QROWS : 0;
  const int seg = lane % L;
  const int rsub = lane / L;

  // Rows are loaded in batches of up to 16 per lane before any is used, so a
  // wave keeps 16 row segments in flight instead of one.
  constexpr int IT = RW / RPI;
  constexpr int B = IT < 16 ? IT : 16;
  const uint32_t w_bytes = VEC ? (uint32_t)(((N - 1) * swn + K) * 2) : 0u;
  const __amdgpu_buffer_rsrc_t rw =
      __builtin_amdgcn_make_buffer_rsrc((void*)w, (short)0, (int)w_bytes, 0x00020000);
  if (active) {
    for (int b0 = 0; b0 < IT; b0 += B) {
      u32x4 raw[B];
#pragma unroll
      for (int i = 0; i < B; ++i) {
        const int row = sub * RW + (b0 + i) * RPI + rsub;
        const int64_t n = n0 + row;
        if constexpr (VEC) {
          // rows past N read zeros (buffer range check)
          // 32-bit offsets: the host routes only weights below 2^31 bytes here
          const uint32_t off = n < N ? ((uint32_t)n * (uint32_t)swn + (uint32_t)(g * G + seg * 8)) * 2u
                                     : 0x80000000u;
          // non-temporal (cache policy bit 1): every weight byte is read
          // once (block 64.4 -> 61.8 us against the default policy)
          raw[i] = __builtin_amdgcn_raw_buffer_load_b128(rw, off, 0, 2);
        } else {
          uint16_t e[8];
#pragma unroll
          for (int j = 0; j < 8; ++j) e[j] = n < N ? w[n * swn + (g * G + seg * 8 + j) * swk] : (uint16_t)0;
          raw[i] = u32x4{e[0] | ((uint32_t)e[1] << 16), e[2] | ((uint32_t)e[3] << 16),
                         e[4] | ((uint32_t)e[5] << 16), e[6] | ((uint32_t)e[7] << 16)};
        }
      }
      // NaN-propagating extremes: a group without NaN takes the reciprocal
      // packing, redone exactly for the rare flagged words; a group with a
      // NaN (NaN extremes) takes the exact path (the sign of a zero extreme
      // does not reach group_stats' result)
#pragma unroll
      for (int i = 0; i < B; ++i) {
        const int row = sub * RW + (b0 + i) * RPI + rsub;
        float v[8];
        unpack_row8<DT>(raw[i], v);
        float mx = fmax_p(v[0], v[1]), mn = fmin_p(v[0], v[1]);
#pragma unroll
        for (int j = 2; j < 8; ++j) {
          mx = fmax_p(mx, v[j]);
          mn = fmin_p(mn, v[j]);
        }
        group_minmax<L>(mx, mn);
        float rcp;
        const QStats st = group_stats_fast(mx, mn, &rcp);
        bool near;
        uint32_t word = quantize_pack8_fast(v, st, rcp, &near);
        // a NaN in the group, a word near a rounding boundary, an infinite
        // scale (infinite weight) or a scale rounded to 0 in fp16: exact path
        if (!(mx == mx && mn == mn) || near || !(st.scale > 0.0f && st.scale < __builtin_inff()))
          word = quantize_pack8(v, st);
        tile[ts][seg][row] = word;
        if (seg == 0) {
          st_s[ts][row] = scale_bits(st.scale);
          st_z[ts][row] = zero_bits(st.zero);
        }
      }
    }
  }
  __syncthreads();
  if (active) {
    const int64_t n = n0 + lane;
    if (n < N) {
      const int64_t k8_0 = g * L;
#pragma unroll 4
      // non-temporal stores: nothing here reads the packed outputs again
      // (3.5 % on the block against cached stores)
      for (int kk = sub; kk < L; kk += WPT)
        __builtin_nontemporal_store((int32_t)tile[ts][kk][lane], &qw[(k8_0 + kk) * N + n]);
      if (sub == 0) {
        __builtin_nontemporal_store(st_s[ts][lane], &sc[g * N + n]);
        __builtin_nontemporal_store(st_z[ts][lane], &ze[g * N + n]);
      }
    }
  }
}

template <int DT, int G, bool VEC>
__global__ __launch_bounds__(QSWAVES * 64) void quantize_small_group_kernel(QuantArgs qa) {
  quantize_small_group_tiles<DT, G, VEC>(qa, (int)blockIdx.x);
}

// Several weights in one launch: workgroup b belongs to the weight whose
// workgroup range holds it (the ranges follow each other in order).
template <int DT, int G>
__global__ __launch_bounds__(QSWAVES * 64) void quantize_small_group_grouped_kernel(QuantGroupedArgs ga) {
  const int b = blockIdx.x;
  int p = 0;
#pragma unroll
  for (int i = 1; i < kQuantMaxGrouped; ++i)
    if (i < ga.count && b >= ga.wg_start[i]) p = i;
  quantize_small_group_tiles<DT, G, true>(ga.prob[p], b - ga.wg_start[p]);
}

// Two-pass kernel for G > 512 (per-channel G = K included): pass 1 reduces
// min/max over the whole group row by row, pass 2 re-reads 512-wide chunks
// and packs them.  One wave per (group, 64-column strip).
template <int DT, bool VEC>
__global__ __launch_bounds__(QWAVES * 64) void quantize_large_group_kernel(
    const uint16_t* __restrict__ w, int64_t N, int64_t K, int64_t swn, int64_t swk, int G,
    int32_t* __restrict__ qw, uint16_t* __restrict__ sc, uint16_t* __restrict__ ze,
    int64_t tiles_n, int64_t tiles_total) {
  __shared__ uint32_t tile[QWAVES][64][QROWS + 1];
  __shared__ float st_scale[QWAVES][QROWS];
  __shared__ float st_zero[QWAVES][QROWS];

  const int lane = threadIdx.x & 63;
  const int wv = threadIdx.x >> 6;
  const int64_t t = (int64_t)blockIdx.x * QWAVES + wv;
  const bool active = t < tiles_total;
  const int64_t g = active ? t / tiles_n : 0;
  const int64_t n0 = active ? (t % tiles_n) * QROWS : 0;
  const int nchunks = G / 512;

  if (active) {
    for (int row = 0; row < QROWS; ++row) {
      const int64_t n = n0 + row;
      if (n >= N) break;
      float mx = 0.0f, mn = 0.0f;
      bool first = true;
      for (int c = 0; c < nchunks; ++c) {
        float v[8];
        load8<DT, VEC>(w, n, g * G + c * 512 + lane * 8, swn, swk, v);
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          mx = first ? v[i] : max_nan(mx, v[i]);
          mn = first ? v[i] : min_nan(mn, v[i]);
          first = false;
        }
      }
#pragma unroll
      for (int off = 32; off > 0; off >>= 1) {
        mx = max_nan(mx, __shfl_xor(mx, off, 64));
        mn = min_nan(mn, __shfl_xor(mn, off, 64));
      }
      const QStats st = group_stats(mx, mn);
      if (lane == 0) {
        st_scale[wv][row] = st.scale;
        st_zero[wv][row] = st.zero;
      }
    }
  }
  __syncthreads();
  if (active) {
    const int64_t n = n0 + lane;
    if (n < N) {
      sc[g * N + n] = scale_bits(st_scale[wv][lane]);
      ze[g * N + n] = zero_bits(st_zero[wv][lane]);
    }
  }
  for (int c = 0; c < nchunks; ++c) {
    if (active) {
      for (int row = 0; row < QROWS; ++row) {
        const int64_t n = n0 + row;
        if (n >= N) break;
        float v[8];
        load8<DT, VEC>(w, n, g * G + c * 512 + lane * 8, swn, swk, v);
        QStats st;
        st.scale = st_scale[wv][row];
        st.zero = st_zero[wv][row];
        tile[wv][lane][row] = quantize_pack8(v, st);
      }
    }
    __syncthreads();
    if (active) {
      const int64_t n = n0 + lane;
      if (n < N) {
        const int64_t k8_0 = g * (G / 8) + (int64_t)c * 64;
        for (int kk = 0; kk < 64; ++kk) qw[(k8_0 + kk) * N + n] = (int32_t)tile[wv][kk][lane];
      }
    }
    __syncthreads();
  }
}

// W_hat[N, K] = round_once((q - z) * s): 64x64-word tiles transposed through
// LDS so that both the qweight reads and the W_hat row writes are coalesced.
template <int ODT>
__global__ __launch_bounds__(256) void dequantize_kernel(const int32_t* __restrict__ qw,
                                                         const uint16_t* __restrict__ sc,
                                                         const uint16_t* __restrict__ ze,
                                                         int64_t N, int64_t K8, int gshift,
                                                         void* __restrict__ out) {
#pragma clang fp contract(off)
  __shared__ uint32_t tile[64][65];
  const int t = threadIdx.x;
  const int64_t n0 = (int64_t)blockIdx.x * 64;
  const int64_t k80 = (int64_t)blockIdx.y * 64;
#pragma unroll 4
  for (int i = 0; i < 16; ++i) {
    const int kk = i * 4 + (t >> 6), nn = t & 63;
    const int64_t k8 = k80 + kk, n = n0 + nn;
    tile[kk][nn] = (k8 < K8 && n < N) ? (uint32_t)qw[k8 * N + n] : 0u;
  }
  __syncthreads();
  const int64_t K = K8 * 8;
#pragma unroll 2
  for (int i = 0; i < 16; ++i) {
    const int nn = i * 4 + (t >> 6), kk = t & 63;
    const int64_t k8 = k80 + kk, n = n0 + nn;
    if (k8 >= K8 || n >= N) continue;
    const uint32_t word = tile[kk][nn];
    const int64_t g = (k8 * 8) >> gshift;
    const float s = half_bits_to_float(sc[g * N + n]);
    const float z = half_bits_to_float(ze[g * N + n]);
    float v[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      v[j] = ((float)((word >> (4 * j)) & 0xFu) - z) * s;
      // Materialize the fp32 product: without this the backend folds
      // multiply + fp16 cast into one mixed fma with a +0 addend, which
      // turns a -0 product (q < z, s = 0) into +0.
      asm volatile("" : "+v"(v[j]));
    }
    if constexpr (ODT == W4_DTYPE_FP32) {
      float* o = reinterpret_cast<float*>(out) + n * K + k8 * 8;
      f32x4 a, b;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        a[j] = v[j];
        b[j] = v[4 + j];
      }
      *reinterpret_cast<f32x4*>(o) = a;
      *reinterpret_cast<f32x4*>(o + 4) = b;
    } else {
      uint16_t* o = reinterpret_cast<uint16_t*>(out) + n * K + k8 * 8;
      u32x4 p;
#pragma unroll
      for (int j = 0; j < 4; ++j)
        p[j] = (uint32_t)float_to_act_bits<ODT>(v[2 * j]) |
               ((uint32_t)float_to_act_bits<ODT>(v[2 * j + 1]) << 16);
      *reinterpret_cast<u32x4*>(o) = p;
    }
  }
}

}  // namespace w4

using namespace w4host;

template <int DT, bool VEC>
static void launch_quantize(const uint16_t* w, int64_t N, int64_t K, int64_t swn, int64_t swk,
                            int G, int32_t* qw, uint16_t* sc, uint16_t* ze, hipStream_t st) {
  const int64_t tiles_n = (N + w4::QROWS - 1) / w4::QROWS;
  const int64_t tiles_total = tiles_n * (K / G);
  const bool small = G <= 512;
  const int64_t tpb = small ? w4::QSWAVES / w4::quantize_waves_per_tile(G) : w4::QWAVES;
  const dim3 grid((unsigned)((tiles_total + tpb - 1) / tpb));
  const dim3 block((small ? w4::QSWAVES : w4::QWAVES) * 64);
  const w4::QuantArgs qa{w, qw, sc, ze, N, K, swn, swk, tiles_n, tiles_total};
#define W4_QS(GG)                                                                                  \
  case GG:                                                                                         \
    hipLaunchKernelGGL((w4::quantize_small_group_kernel<DT, GG, VEC>), grid, block, 0, st, qa); \
    return;
  switch (G) {
    W4_QS(8)
    W4_QS(16)
    W4_QS(32)
    W4_QS(64)
    W4_QS(128)
    W4_QS(256)
    W4_QS(512)
    default:
      break;
  }
#undef W4_QS
  hipLaunchKernelGGL((w4::quantize_large_group_kernel<DT, VEC>), grid, block, 0, st, w, N, K, swn,
                     swk, G, qw, sc, ze, tiles_n, tiles_total);
}

extern "C" int w4_quantize(const void* w, int w_dtype, int64_t N, int64_t K, int64_t stride_wn,
                           int64_t stride_wk, int group_size, int32_t* qweight, uint16_t* scales,
                           uint16_t* zeros, void* stream) {
  clear_error();
  if (w_dtype != W4_DTYPE_BF16 && w_dtype != W4_DTYPE_FP16)
    return fail(W4_ERR_INVALID, "w4_quantize: weight dtype must be bf16 or fp16 (got code %d)", w_dtype);
  if (N < 0 || K <= 0) return fail(W4_ERR_INVALID, "w4_quantize: bad shape N=%lld K=%lld", (long long)N, (long long)K);
  const int64_t G = group_size == -1 ? K : group_size;
  if (G <= 0 || K % G != 0 || G % 8 != 0 || !is_pow2(G))
    return fail(W4_ERR_INVALID,
                "w4_quantize: group_size must be a power of two, a multiple of 8 and divide K "
                "(K=%lld, group_size=%d)", (long long)K, group_size);
  if (G > (int64_t)1 << 30) return fail(W4_ERR_UNSUPPORTED, "w4_quantize: group_size too large");
  if (N == 0) return W4_OK;
  if (!w || !qweight || !scales || !zeros) return fail(W4_ERR_INVALID, "w4_quantize: null pointer");
  if (((N + 63) / 64) * (K / G) >= (int64_t)1 << 31)
    return fail(W4_ERR_UNSUPPORTED, "w4_quantize: %lld x %lld weight has too many tiles", (long long)N,
                (long long)K);
  const uint16_t* wp = static_cast<const uint16_t*>(w);
  // 128-bit buffer loads: dense rows, 16-byte aligned, whole tensor within 2 GiB
  const bool vec = stride_wk == 1 && (stride_wn % 8) == 0 && ((uintptr_t)wp % 16) == 0 &&
                   ((N - 1) * stride_wn + K) * 2 < (1LL << 31);
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (w_dtype == W4_DTYPE_BF16) {
    if (vec) launch_quantize<W4_DTYPE_BF16, true>(wp, N, K, stride_wn, stride_wk, (int)G, qweight, scales, zeros, st);
    else launch_quantize<W4_DTYPE_BF16, false>(wp, N, K, stride_wn, stride_wk, (int)G, qweight, scales, zeros, st);
  } else {
    if (vec) launch_quantize<W4_DTYPE_FP16, true>(wp, N, K, stride_wn, stride_wk, (int)G, qweight, scales, zeros, st);
    else launch_quantize<W4_DTYPE_FP16, false>(wp, N, K, stride_wn, stride_wk, (int)G, qweight, scales, zeros, st);
  }
  return check_launch("w4_quantize");
}

// One grouped launch when every weight takes the single-pass 128-bit path
// with the same group size; otherwise one w4_quantize per weight, in order.
extern "C" int w4_quantize_grouped(const w4_quantize_problem* problems, int count, int w_dtype, void* stream) {
  clear_error();
  if (count < 1 || count > W4_MAX_GROUPED)
    return fail(W4_ERR_INVALID, "w4_quantize_grouped: count must be in [1, %d]", W4_MAX_GROUPED);
  if (!problems) return fail(W4_ERR_INVALID, "w4_quantize_grouped: null problem list");
  if (w_dtype != W4_DTYPE_BF16 && w_dtype != W4_DTYPE_FP16)
    return fail(W4_ERR_INVALID, "w4_quantize_grouped: weight dtype must be bf16 or fp16 (got code %d)", w_dtype);
  static_assert(W4_MAX_GROUPED <= w4::kQuantMaxGrouped, "grouped quantize capacity");
  w4::QuantGroupedArgs ga{};
  int64_t G0 = -1, wgs = 0;
  bool one_launch = true;
  for (int i = 0; i < count; ++i) {
    const w4_quantize_problem& q = problems[i];
    if (q.N < 0 || q.K <= 0)
      return fail(W4_ERR_INVALID, "w4_quantize_grouped: bad shape in problem %d (N=%lld K=%lld)", i,
                  (long long)q.N, (long long)q.K);
    const int64_t G = q.group_size == -1 ? q.K : q.group_size;
    if (G <= 0 || q.K % G != 0 || G % 8 != 0 || !is_pow2(G))
      return fail(W4_ERR_INVALID, "w4_quantize_grouped: bad group size %d in problem %d (K=%lld)", q.group_size, i,
                  (long long)q.K);
    if (q.N > 0 && (!q.w || !q.qweight || !q.scales || !q.zeros))
      return fail(W4_ERR_INVALID, "w4_quantize_grouped: null pointer in problem %d", i);
    const bool vec = q.stride_wk == 1 && (q.stride_wn % 8) == 0 && ((uintptr_t)q.w % 16) == 0 &&
                     ((q.N - 1) * q.stride_wn + q.K) * 2 < (1LL << 31) && ((q.N + 63) / 64) * (q.K / G) < (1LL << 30);
    one_launch = one_launch && q.N > 0 && vec && G <= 512 && (G0 < 0 || G == G0);
    G0 = G;
    if (!one_launch) continue;
    const int64_t tiles_n = (q.N + w4::QROWS - 1) / w4::QROWS, tiles_total = tiles_n * (q.K / G);
    const int64_t tpb = w4::QSWAVES / w4::quantize_waves_per_tile((int)G);
    ga.prob[i] = w4::QuantArgs{static_cast<const uint16_t*>(q.w), q.qweight, q.scales, q.zeros, q.N, q.K,
                               q.stride_wn, q.stride_wk, tiles_n, tiles_total};
    ga.wg_start[i] = (int)wgs;
    wgs += (tiles_total + tpb - 1) / tpb;
    one_launch = wgs < (1LL << 30);
  }
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (!one_launch) {
    for (int i = 0; i < count; ++i) {
      const w4_quantize_problem& q = problems[i];
      const int rc = w4_quantize(q.w, w_dtype, q.N, q.K, q.stride_wn, q.stride_wk, q.group_size, q.qweight,
                                 q.scales, q.zeros, stream);
      if (rc != W4_OK) return rc;
    }
    return W4_OK;
  }
  for (int i = count; i <= w4::kQuantMaxGrouped; ++i) ga.wg_start[i] = (int)wgs;
  ga.count = count;
  const dim3 grid((unsigned)wgs), block(w4::QSWAVES * 64);
#define W4_QG(DT, GG)                                                                                \
  case GG:                                                                                           \
    hipLaunchKernelGGL((w4::quantize_small_group_grouped_kernel<DT, GG>), grid, block, 0, st, ga); \
    break;
  if (w_dtype == W4_DTYPE_BF16) {
    switch (G0) { W4_QG(W4_DTYPE_BF16, 8) W4_QG(W4_DTYPE_BF16, 16) W4_QG(W4_DTYPE_BF16, 32) W4_QG(W4_DTYPE_BF16, 64)
                  W4_QG(W4_DTYPE_BF16, 128) W4_QG(W4_DTYPE_BF16, 256) W4_QG(W4_DTYPE_BF16, 512) default: break; }
  } else {
    switch (G0) { W4_QG(W4_DTYPE_FP16, 8) W4_QG(W4_DTYPE_FP16, 16) W4_QG(W4_DTYPE_FP16, 32) W4_QG(W4_DTYPE_FP16, 64)
                  W4_QG(W4_DTYPE_FP16, 128) W4_QG(W4_DTYPE_FP16, 256) W4_QG(W4_DTYPE_FP16, 512) default: break; }
  }
#undef W4_QG
  return check_launch("w4_quantize_grouped");
}

extern "C" int w4_dequantize(const int32_t* qweight, const uint16_t* scales, const uint16_t* zeros,
                             int64_t N, int64_t K, int group_size, int out_dtype, void* out,
                             void* stream) {
  clear_error();
  if (N < 0 || K <= 0 || K % 8 != 0)
    return fail(W4_ERR_INVALID, "w4_dequantize: bad shape N=%lld K=%lld", (long long)N, (long long)K);
  const int64_t G = group_size == -1 ? K : group_size;
  if (G <= 0 || K % G != 0 || G % 8 != 0 || !is_pow2(G))
    return fail(W4_ERR_INVALID, "w4_dequantize: bad group_size %d for K=%lld", group_size, (long long)K);
  if (N == 0) return W4_OK;
  if (!qweight || !scales || !zeros || !out) return fail(W4_ERR_INVALID, "w4_dequantize: null pointer");
  if (((uintptr_t)out % 16) != 0) return fail(W4_ERR_INVALID, "w4_dequantize: output must be 16-byte aligned");
  const int64_t K8 = K / 8;
  const dim3 grid((unsigned)((N + 63) / 64), (unsigned)((K8 + 63) / 64));
  const int gshift = ilog2(G);
  hipStream_t st = static_cast<hipStream_t>(stream);
  switch (out_dtype) {
    case W4_DTYPE_BF16:
      hipLaunchKernelGGL((w4::dequantize_kernel<W4_DTYPE_BF16>), grid, dim3(256), 0, st, qweight, scales, zeros, N, K8, gshift, out);
      break;
    case W4_DTYPE_FP16:
      hipLaunchKernelGGL((w4::dequantize_kernel<W4_DTYPE_FP16>), grid, dim3(256), 0, st, qweight, scales, zeros, N, K8, gshift, out);
      break;
    case W4_DTYPE_FP32:
      hipLaunchKernelGGL((w4::dequantize_kernel<W4_DTYPE_FP32>), grid, dim3(256), 0, st, qweight, scales, zeros, N, K8, gshift, out);
      break;
    default:
      return fail(W4_ERR_INVALID, "w4_dequantize: bad out dtype %d", out_dtype);
  }
  return check_launch("w4_dequantize");
}
