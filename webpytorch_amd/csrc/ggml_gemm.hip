// GGUF K-quant prefill GEMM on the gfx950 matrix cores: out[m][n] = x[m][:] . W[n][:] (+ bias[n])
// for many activation rows, W = N rows of blocks as the file stores them, for the four types of
// a Q4_K_M / Q5_K_M file: Q4_K, Q5_K, Q6_K and Q8_0 (8 consecutive 32-value blocks make one
// 256-value step). Block layouts (llama.cpp's):
//   Q4_K (144 bytes): fp16 d, fp16 dmin, 12 bytes of 6-bit scales/mins, qs[128];
//   Q5_K (176 bytes): the same header, qh[32], qs[128] -- the fifth bit of value l of
//     sub-block j is bit j of qh[l];
//   Q6_K (210 bytes): ql[128], qh[64], 16 int8 scales, fp16 d -- value 128 h + 32 j + l has code
//     ((ql[64 h + 32 (j & 1) + l] >> 4 (j >> 1)) & 15) | ((qh[32 h + l] >> 2 j) & 3) << 4 and
//     scale byte 8 h + 2 j + l / 16;
//   Q8_0 (34 bytes): fp16 d, 32 int8 codes.
//
// Every product runs on the fp16 matrix cores with an exact integer B operand:
//   * Q4_K / Q5_K: a sub-block of 32 weights holds w = d sc c - dmin m, so per sub-block
//     sum_k x_k w_k = d (sc sum_k x_k c_k) - dmin (m sum_k x_k); B = sc c is an integer below
//     2048 (63 x 31 at most), exact in fp16, so the eight sub-blocks chain in one accumulator;
//     the row sums of x come precomputed per sub-block and the mins multiply them on the fp32
//     matrix cores; d and dmin apply once per super-block.
//   * Q6_K: w = d sc (c - 32) with a signed 8-bit sc and 16-value sub-blocks, so (c - 32) sc
//     (up to 4096) is not exact in fp16; sc = 16 sh + sl (sl = sc & 15, sh = sc >> 4) splits it
//     into two exact operands, (c - 32) sl and (c - 32) 16 sh, two MFMAs into one accumulator;
//     d applies once per super-block.
//   * Q8_0: B = q (int8, exact); each 32-value block has its own d, so every block's product
//     starts from zero and is folded into the accumulator as d P (four fp32 FMAs per tile).
// Codes become fp16 operands by OR-ing them into the mantissa of 1024.0 and subtracting 1024
// (plus the code offset), no conversion instruction per code.
//
// fp32 activations enter as two fp16 rows each, hi = fp16(x 2^s) and lo = fp16(x 2^s - hi),
// with 2^s per row putting the row's largest |x| near 2^15 (s = 0 for rows holding NaN or Inf);
// the staging pass writes them and their sub-block sums as rows 2m and 2m + 1, and the GEMM's
// epilogue adds the pair and scales back. fp16 activations are staged as they are.
//
// Staged rows: xs[r][k] fp16, each 8-wide k block in the order (0, 2, 1, 3, 4, 6, 5, 7) that
// the code unpack produces (byte j of a code word holds value j, and one v_and_or_b32 takes
// bytes 0 and 2, then 1 and 3); rs[r][k / 32] the sub-block sums of the staged fp16 values
// (fp32).
//
// Tiles: a workgroup of 4 waves computes 64 rows x 64 CG columns; wave w takes the CG groups of
// 16 columns from 16 CG w and all 64 rows (four 16-row MFMA tiles per group). K is walked 256
// weights at a time: the 64 x 256 activation tile sits in LDS (16-byte chunks XOR-swizzled by
// row, so the 16 rows that one operand read touches fall in different banks) and each lane holds
// the block bytes of its column and its 8-value k runs in registers, loaded one step ahead.
// Workgroups are ordered XCD-major with row tiles fastest, so the row tiles of a column tile
// share that XCD's L2.
//
// Block starts: Q4_K and Q5_K blocks are 16-byte aligned, as are Q8_0's 272-byte steps; Q6_K
// blocks are only 2-byte aligned (210 bytes), so its loads are dwords at the rounded-down
// address, realigned with v_alignbyte, and never reach past the block (details at load_raw).
#include <math.h>

#include <algorithm>
#include <type_traits>

#include "miq_common.h"

namespace miq {
namespace kg {

constexpr int kXCDs = 8;
constexpr int kBM = 64;
constexpr int kCUs = 256;

typedef _Float16 half8v __attribute__((ext_vector_type(8)));
typedef float float4v __attribute__((ext_vector_type(4)));

__device__ __forceinline__ int row_exp(float m) {
  if (!(m > 0.f) || !(m <= 3.4e38f)) return 0;
  int ex;
  frexpf(m, &ex);
  return min(max(15 - ex, -126), 126);  // any finite maximum lands below 2^15; 2^s stays finite
}

// fp16 pair (a, b) as one word
__device__ __forceinline__ uint32_t h2(__half a, __half b) {
  return (uint32_t)__half_as_ushort(a) | ((uint32_t)__half_as_ushort(b) << 16);
}
// 8 fp16 values of k order into the unpack's order (0, 2, 1, 3, 4, 6, 5, 7), as 4 words
__device__ __forceinline__ uint4 order8(const __half* h) {
  return make_uint4(h2(h[0], h[2]), h2(h[1], h[3]), h2(h[4], h[6]), h2(h[5], h[7]));
}
__device__ __forceinline__ float sum8(const __half* h) {
  return ((__half2float(h[0]) + __half2float(h[1])) + (__half2float(h[2]) + __half2float(h[3]))) +
         ((__half2float(h[4]) + __half2float(h[5])) + (__half2float(h[6]) + __half2float(h[7])));
}

// One workgroup per row m of x: rows R m .. R m + R - 1 of xs (R = 2 for fp32 x: hi, lo; 1 for
// fp16) with their sub-block sums, and for fp32 the row's largest |x| (NaN if it holds one) in
// rmax[m]. The four threads of a sub-block are consecutive (quad), so its sum is a quad sum.
// Dynamic LDS K * 4 bytes for fp32 (the row is read once, its maximum sets the scale).
template <typename XT>
__global__ __launch_bounds__(256) void stage_kernel(const XT* __restrict__ x, __half* __restrict__ xs,
                                                    float* __restrict__ rs, float* __restrict__ rmax, int K) {
  constexpr bool F32 = std::is_same<XT, float>::value;
  const int m = blockIdx.x, nch = K / 8, K32 = K / 32;
  float sc = 1.f;
  extern __shared__ __align__(16) float frow[];
  if constexpr (F32) {
    __shared__ float wmax[4];
    __shared__ int wnan[4];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const float* src = x + (size_t)m * K;
    float mx = 0.f;
    bool nan = false;
#pragma unroll 4
    for (int q = threadIdx.x; q < K / 4; q += 256) {
      const float4 v = reinterpret_cast<const float4*>(src)[q];
      reinterpret_cast<float4*>(frow)[q] = v;
      mx = fmaxf(mx, fmaxf(fmaxf(fabsf(v.x), fabsf(v.y)), fmaxf(fabsf(v.z), fabsf(v.w))));
      nan |= v.x != v.x || v.y != v.y || v.z != v.z || v.w != v.w;
    }
    nan = __ballot(nan) != 0ull;
    mx = wave_max(mx);
    if (lane == 0) {
      wmax[wave] = mx;
      wnan[wave] = nan;
    }
    __syncthreads();
    mx = fmaxf(fmaxf(wmax[0], wmax[1]), fmaxf(wmax[2], wmax[3]));
    if (wnan[0] | wnan[1] | wnan[2] | wnan[3]) mx = __int_as_float(0x7FC00000);
    if (threadIdx.x == 0) rmax[m] = mx;
    sc = ldexpf(1.f, row_exp(mx));
  }
  for (int i = threadIdx.x; i < nch; i += 256) {  // nch is a multiple of 32: quads stay whole
    __half hi[8], lo[8];
    if constexpr (F32) {
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const float a = frow[8 * i + j] * sc;
        hi[j] = __float2half_rn(a);
        lo[j] = __float2half_rn(a - __half2float(hi[j]));
      }
    } else {
      const uint4 v = *reinterpret_cast<const uint4*>(x + (size_t)m * K + 8 * i);
      const uint32_t wv[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        hi[2 * j] = __ushort_as_half((unsigned short)(wv[j] & 0xFFFFu));
        hi[2 * j + 1] = __ushort_as_half((unsigned short)(wv[j] >> 16));
      }
    }
    constexpr int R = F32 ? 2 : 1;
    *reinterpret_cast<uint4*>(xs + ((size_t)R * m) * K + 8 * i) = order8(hi);
    const float shi = quad_sum(sum8(hi));
    if ((i & 3) == 0) rs[((size_t)R * m) * K32 + i / 4] = shi;
    if constexpr (F32) {
      *reinterpret_cast<uint4*>(xs + ((size_t)R * m + 1) * K + 8 * i) = order8(lo);
      const float slo = quad_sum(sum8(lo));
      if ((i & 3) == 0) rs[((size_t)R * m + 1) * K32 + i / 4] = slo;
    }
  }
}

// ggml type ids of the four types
constexpr int kQ8_0 = 8, kQ4_K = 12, kQ5_K = 13, kQ6_K = 14;

// Per type: bytes per 256-value step, raw 32-bit registers per lane and step, whether the
// sub-block mins (and so the row sums) enter.
template <int T> struct KQ;
template <> struct KQ<kQ4_K> { static constexpr int STEP = 144, RAW = 12; static constexpr bool MIN = true; };
template <> struct KQ<kQ5_K> { static constexpr int STEP = 176, RAW = 14; static constexpr bool MIN = true; };
template <> struct KQ<kQ6_K> { static constexpr int STEP = 210, RAW = 24; static constexpr bool MIN = false; };
template <> struct KQ<kQ8_0> { static constexpr int STEP = 272, RAW = 32; static constexpr bool MIN = false; };

__device__ __forceinline__ uint32_t ld32(const uint8_t* p) { return *reinterpret_cast<const uint32_t*>(p); }
__device__ __forceinline__ uint32_t ld16(const uint8_t* p) { return *reinterpret_cast<const unsigned short*>(p); }

// The bytes lane (column, kb) needs from one 256-value step at bp: for each 32-value sub-block
// the 8 codes of values 8 kb .. 8 kb + 7, plus the step's scales.
//   Q4_K: r[0..3] header (d, dmin, scales), r[4 + 2g], r[5 + 2g] qs[32 g + 8 kb ..] (g < 4:
//         sub-blocks 2g in the low nibbles, 2g + 1 in the high ones).
//   Q5_K: the same with qs at byte 48, and r[12..13] qh[8 kb ..].
//   Q6_K: bp % 4 = s is 0 or 2 and the same for every piece (all offsets are multiples of 4):
//         each 8-byte piece at a is three dwords from a - s (the last ends at a + 12 - s, at most
//         byte 196 of the block); pieces ql[64 h + 32 e + 8 kb ..] (i = 2h + e) at r[3i..],
//         qh[32 h + 8 kb ..] at r[12 + 3h..]; the 16 scale bytes as dwords from 192 - s, the
//         fifth (needed only for s = 2) at 208 - s, else a repeat of the fourth, so no read
//         passes byte 209; d (fp16 at 208) in r[23]. A read at a - s < a stays in the previous
//         block of the row or of the row before, and the weight buffer starts 4-byte aligned.
//   Q8_0: bp is 16-byte aligned (weights 16-byte aligned, rows of 272-byte steps); block b's
//         codes for kb sit at a = 34 b + 2 + 8 kb, 4-byte aligned for odd b (two dwords) and
//         2-byte aligned for even b (dwords at a - 2 and a + 2 and the 2 bytes at a + 6, ending
//         at the block's last code byte); d of block b (fp16 at 34 b) in r[4b + 3].
template <int T> __device__ __forceinline__ void load_raw(const uint8_t* bp, int kb, uint32_t* r) {
  if constexpr (T == kQ4_K || T == kQ5_K) {
    const uint4 h = *reinterpret_cast<const uint4*>(bp);
    r[0] = h.x; r[1] = h.y; r[2] = h.z; r[3] = h.w;
    constexpr int QS = T == kQ4_K ? 16 : 48;
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      const uint2 c = *reinterpret_cast<const uint2*>(bp + QS + 32 * g + 8 * kb);
      r[4 + 2 * g] = c.x;
      r[5 + 2 * g] = c.y;
    }
    if constexpr (T == kQ5_K) {
      const uint2 c = *reinterpret_cast<const uint2*>(bp + 16 + 8 * kb);
      r[12] = c.x;
      r[13] = c.y;
    }
  } else if constexpr (T == kQ6_K) {
    const int s = (int)(reinterpret_cast<uintptr_t>(bp) & 3);
    const uint8_t* b4 = bp - s;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const uint8_t* q = b4 + 64 * (i >> 1) + 32 * (i & 1) + 8 * kb;
      r[3 * i] = ld32(q); r[3 * i + 1] = ld32(q + 4); r[3 * i + 2] = ld32(q + 8);
    }
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const uint8_t* q = b4 + 128 + 32 * h + 8 * kb;
      r[12 + 3 * h] = ld32(q); r[13 + 3 * h] = ld32(q + 4); r[14 + 3 * h] = ld32(q + 8);
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) r[18 + i] = ld32(b4 + 192 + 4 * i);
    r[22] = ld32(b4 + (s ? 208 : 204));
    r[23] = ld16(bp + 208);
  } else {
#pragma unroll
    for (int b = 0; b < 8; ++b) {
      const uint8_t* q = bp + 34 * b + 2 + 8 * kb;
      if (b & 1) {
        r[4 * b] = ld32(q); r[4 * b + 1] = ld32(q + 4); r[4 * b + 2] = 0u;
      } else {
        r[4 * b] = ld32(q - 2); r[4 * b + 1] = ld32(q + 2); r[4 * b + 2] = ld16(q + 6);
      }
      r[4 * b + 3] = ld16(bp + 34 * b);
    }
  }
}

// The 6-bit scale and min of sub-block j from the 12 packed bytes (words s0, s1, s2 = bytes
// 0-3, 4-7, 8-11).
__device__ __forceinline__ void scale_min(uint32_t s0, uint32_t s1, uint32_t s2, int j, uint32_t* sc, uint32_t* mn) {
  const uint32_t q[3] = {s0, s1, s2};
  auto byte = [&](int b) { return (q[b >> 2] >> (8 * (b & 3))) & 0xFFu; };
  if (j < 4) {
    *sc = byte(j) & 63u;
    *mn = byte(j + 4) & 63u;
  } else {
    *sc = (byte(j + 4) & 15u) | ((byte(j - 4) >> 6) << 4);
    *mn = (byte(j + 4) >> 4) | ((byte(j) >> 6) << 4);
  }
}

// Codes in the low M bits of bytes 0-3 of w0 and 4-7 of w1 (the bits above masked off) as the
// fp16 B fragment in the unpack's order, each minus `off`.
template <uint32_t MASK>
__device__ __forceinline__ half8v b_codes(uint32_t w0, uint32_t w1, _Float16 off) {
  const half2v k = (half2v){(_Float16)1024 + off, (_Float16)1024 + off};
  constexpr uint32_t m = MASK | (MASK << 16);
  const half2v a = as_h2(and_or(w0, m, 0x64006400u)) - k;
  const half2v b = as_h2(and_or(w0 >> 8, m, 0x64006400u)) - k;
  const half2v c = as_h2(and_or(w1, m, 0x64006400u)) - k;
  const half2v d = as_h2(and_or(w1 >> 8, m, 0x64006400u)) - k;
  return (half8v){a[0], a[1], b[0], b[1], c[0], c[1], d[0], d[1]};
}

__device__ __forceinline__ float f16f(uint32_t u) { return __half2float(__ushort_as_half((unsigned short)(u & 0xFFFFu))); }

// y[r][n] for rows r < Mx of xs, W of type T. Grid (ntiles * mtiles), 256 threads.
//
// Per 256-value step (see the file comment for the per-type products): the activation tile and
// (Q4_K / Q5_K) the row sums arrive by LDS DMA into one of two buffers while the other is
// multiplied (the swizzle is applied on the source side: DMA lane l of a 1 KB block lands at
// slot l); each lane's block bytes are loaded into registers one step ahead. Q4_K / Q5_K:
// P = sum_sb sc_sb (x . c_sb) on the fp16 matrix cores, Q = sum_sb m_sb rs_sb on the fp32
// matrix cores (two v_mfma_f32_16x16x4_f32: A the row sums, B the column's 6-bit mins), then
// acc += d P - dmin Q. The output (+ bias[n]) as OT. fp16 rows (PAIR false): y[row][n] = acc.
// fp32 rows (PAIR true): staged rows 2m and 2m + 1 are the hi and lo planes of row m, held by
// the same lane (rows 4 kb + r of a 16-row tile), so y[m][n] = (acc[2m] + acc[2m + 1]) 2^-s(m),
// s from rmax[m].
template <int T, int CG, typename OT, bool PAIR>
__global__ __launch_bounds__(256) void gemm_kernel(const __half* __restrict__ xs, const float* __restrict__ rs,
                                                   const uint8_t* __restrict__ w, OT* __restrict__ y,
                                                   const float* __restrict__ bias, const float* __restrict__ rmax,
                                                   int Mx, int K, int N, int mtiles, int tiles, int ksteps,
                                                   float* __restrict__ part) {
  constexpr int RAW = KQ<T>::RAW, STEP = KQ<T>::STEP;
  constexpr bool MIN = KQ<T>::MIN;
  __shared__ __align__(16) __half at[2][kBM * 256];  // activation tiles, 16-byte chunks swizzled by row
  // sub-block sums [sub-block][row], rows of kRT floats: the lanes of one read take rows p and
  // sub-blocks kb, and at 64 floats (256 bytes) per sub-block the four kb share their banks
  constexpr int kRT = kBM + 16;
  __shared__ __align__(16) float rt[MIN ? 2 : 1][MIN ? 8 * kRT : 1];
  const int Tg = (int)gridDim.x, L = (int)blockIdx.x;
  const int Lp = Tg % kXCDs == 0 ? (L % kXCDs) * (Tg / kXCDs) + L / kXCDs : L;
  // K-slice kz of a split product (part != null): steps [s0, s1) of the row, raw sums to part
  const int kz = Lp / tiles, mt = (Lp % tiles) % mtiles, nt = (Lp % tiles) / mtiles;
  const int m0 = mt * kBM, n0 = nt * 64 * CG;
  const int tid = threadIdx.x, lane = tid & 63, wave = uniform(tid >> 6), p = lane & 15, kb = lane >> 4;
  const int nsb = K / 256, K32 = K / 32, s0 = kz * ksteps, s1 = min(nsb, s0 + ksteps);
  // wave w takes the column groups CG w .. CG w + CG - 1 (16 columns each); every operand read
  // of the activation tile feeds one MFMA per group (two for Q6_K)
  int ncol[CG];
  const uint8_t* wr[CG];
#pragma unroll
  for (int c = 0; c < CG; ++c) {
    ncol[c] = n0 + 16 * (CG * wave + c) + p;
    const int n = min(ncol[c], N - 1);  // columns past N repeat the last one and are not stored
    wr[c] = w + (size_t)n * nsb * STEP;
  }

  // this wave's share of the copies of step s into buffer b: 8 of the tile's 32 KB (two rows
  // per 1 KB block) and 2 of its 8 sub-block-sum columns
  auto issue = [&](int s, int b) __attribute__((always_inline)) {
    const uint32_t abase = lds_addr(at[b]);
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int j = wave * 8 + i, r = 2 * j + (lane >> 5), c = (lane & 31) ^ (r & 31);
      dma16(xs + (size_t)min(m0 + r, Mx - 1) * K + s * 256 + c * 8, uniform((int)(abase + j * 1024)));
    }
    if constexpr (MIN) {
      const uint32_t rbase = lds_addr(rt[b]);
#pragma unroll
      for (int i = 0; i < 2; ++i) {
        const int sb = wave * 2 + i;
        dma4(rs + (size_t)min(m0 + lane, Mx - 1) * K32 + s * 8 + sb, uniform((int)(rbase + sb * kRT * 4)));
      }
    }
  };
  uint32_t raw[CG][RAW], nxt[CG][RAW];
  auto load_b = [&](int s) __attribute__((always_inline)) {
#pragma unroll
    for (int c = 0; c < CG; ++c) load_raw<T>(wr[c] + (size_t)s * STEP, kb, nxt[c]);
  };

  float4v acc[CG][4];
#pragma unroll
  for (int c = 0; c < CG; ++c)
#pragma unroll
    for (int t = 0; t < 4; ++t) acc[c][t] = (float4v){0.f, 0.f, 0.f, 0.f};
  issue(s0, s0 & 1);
  load_b(s0);
  for (int s = s0; s < s1; ++s) {
    wait_vmcnt<0>();  // this wave's copies of step s (and its block bytes) have landed
    __syncthreads();  // everyone's copies are in; everyone is done with the other buffer
    if (s + 1 < s1) issue(s + 1, (s + 1) & 1);
#pragma unroll
    for (int c = 0; c < CG; ++c)
#pragma unroll
      for (int i = 0; i < RAW; ++i) raw[c][i] = nxt[c][i];
    if (s + 1 < s1) load_b(s + 1);
    const __half* a = at[s & 1];
    auto afrag = [&](int sb, int t) __attribute__((always_inline)) {
      const int r = 16 * t + p;
      return *reinterpret_cast<const half8v*>(a + r * 256 + (((4 * sb + kb) ^ (r & 31)) * 8));
    };
    if constexpr (T == kQ4_K || T == kQ5_K) {
      float4v P[CG][4], Q[CG][4];
#pragma unroll
      for (int c = 0; c < CG; ++c)
#pragma unroll
        for (int t = 0; t < 4; ++t) P[c][t] = Q[c][t] = (float4v){0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int sb = 0; sb < 8; ++sb) {
        const int sh = 4 * (sb & 1), g = sb >> 1;
        half8v bf[CG];
#pragma unroll
        for (int c = 0; c < CG; ++c) {
          uint32_t sc, mn;
          scale_min(raw[c][1], raw[c][2], raw[c][3], sb, &sc, &mn);
          uint32_t c0 = raw[c][4 + 2 * g] >> sh, c1 = raw[c][5 + 2 * g] >> sh;  // b_codes masks Q4_K's
          if constexpr (T == kQ5_K) {
            c0 = (c0 & 0x0F0F0F0Fu) | (((raw[c][12] >> sb) & 0x01010101u) << 4);
            c1 = (c1 & 0x0F0F0F0Fu) | (((raw[c][13] >> sb) & 0x01010101u) << 4);
          }
          bf[c] = b_codes<T == kQ5_K ? 0x1Fu : 0x0Fu>(c0, c1, (_Float16)0) * (_Float16)(float)sc;
        }
#pragma unroll
        for (int t = 0; t < 4; ++t) {
          const half8v af = afrag(sb, t);
#pragma unroll
          for (int c = 0; c < CG; ++c) P[c][t] = __builtin_amdgcn_mfma_f32_16x16x32_f16(af, bf[c], P[c][t], 0, 0, 0);
        }
      }
      {  // Q = sum over the 8 sub-blocks of rs[row][sb] m[sb][col]: k = kb, then 4 + kb
        const float* r8 = rt[s & 1];
        float m_lo[CG], m_hi[CG];
#pragma unroll
        for (int c = 0; c < CG; ++c) {
          uint32_t sc, mlo, mhi;
          scale_min(raw[c][1], raw[c][2], raw[c][3], kb, &sc, &mlo);
          scale_min(raw[c][1], raw[c][2], raw[c][3], 4 + kb, &sc, &mhi);
          m_lo[c] = (float)mlo;
          m_hi[c] = (float)mhi;
        }
#pragma unroll
        for (int t = 0; t < 4; ++t) {
          const float rlo = r8[kb * kRT + 16 * t + p], rhi = r8[(4 + kb) * kRT + 16 * t + p];
#pragma unroll
          for (int c = 0; c < CG; ++c) {
            Q[c][t] = __builtin_amdgcn_mfma_f32_16x16x4f32(rlo, m_lo[c], Q[c][t], 0, 0, 0);
            Q[c][t] = __builtin_amdgcn_mfma_f32_16x16x4f32(rhi, m_hi[c], Q[c][t], 0, 0, 0);
          }
        }
      }
#pragma unroll
      for (int c = 0; c < CG; ++c) {
        const float d = f16f(raw[c][0]), dmin = f16f(raw[c][0] >> 16);
#pragma unroll
        for (int t = 0; t < 4; ++t)
#pragma unroll
          for (int q = 0; q < 4; ++q) acc[c][t][q] = fmaf(d, P[c][t][q], fmaf(-dmin, Q[c][t][q], acc[c][t][q]));
      }
    } else if constexpr (T == kQ6_K) {
      float4v P[CG][4];
#pragma unroll
      for (int c = 0; c < CG; ++c)
#pragma unroll
        for (int t = 0; t < 4; ++t) P[c][t] = (float4v){0.f, 0.f, 0.f, 0.f};
      uint32_t sa[CG];  // the block's byte offset mod 4 (0 or 2), in bits for v_alignbyte
#pragma unroll
      for (int c = 0; c < CG; ++c) sa[c] = (uint32_t)(reinterpret_cast<uintptr_t>(wr[c] + (size_t)s * STEP) & 3);
#pragma unroll
      for (int sb = 0; sb < 8; ++sb) {
        const int h = sb >> 2, j = sb & 3, i = 2 * h + (j & 1);
        half8v blo[CG], bhi[CG];
#pragma unroll
        for (int c = 0; c < CG; ++c) {
          const uint32_t* R = raw[c];
          const uint32_t q0 = __builtin_amdgcn_alignbyte(R[3 * i + 1], R[3 * i], sa[c]);
          const uint32_t q1 = __builtin_amdgcn_alignbyte(R[3 * i + 2], R[3 * i + 1], sa[c]);
          const uint32_t h0 = __builtin_amdgcn_alignbyte(R[13 + 3 * h], R[12 + 3 * h], sa[c]);
          const uint32_t h1 = __builtin_amdgcn_alignbyte(R[14 + 3 * h], R[13 + 3 * h], sa[c]);
          const int nib = 4 * (j >> 1);
          const uint32_t c0 = ((q0 >> nib) & 0x0F0F0F0Fu) | (((h0 >> (2 * j)) & 0x03030303u) << 4);
          const uint32_t c1 = ((q1 >> nib) & 0x0F0F0F0Fu) | (((h1 >> (2 * j)) & 0x03030303u) << 4);
          const half8v q = b_codes<0x3Fu>(c0, c1, (_Float16)32);  // c - 32, exact
          // scale byte 8 h + 2 j + kb / 2 of the 16 (dwords 18..22 from the rounded-down 192)
          const int e = 8 * h + 2 * j;  // + kb / 2, lane-dependent
          const uint32_t wsc = __builtin_amdgcn_alignbyte(R[18 + (e >> 2) + 1], R[18 + (e >> 2)], sa[c]);
          const int sc = (int)(int8_t)(wsc >> (8 * ((e & 3) + (kb >> 1))));
          blo[c] = q * (_Float16)(float)(sc & 15);
          bhi[c] = q * (_Float16)(float)(16 * (sc >> 4));
        }
#pragma unroll
        for (int t = 0; t < 4; ++t) {
          const half8v af = afrag(sb, t);
#pragma unroll
          for (int c = 0; c < CG; ++c) {
            P[c][t] = __builtin_amdgcn_mfma_f32_16x16x32_f16(af, blo[c], P[c][t], 0, 0, 0);
            P[c][t] = __builtin_amdgcn_mfma_f32_16x16x32_f16(af, bhi[c], P[c][t], 0, 0, 0);
          }
        }
      }
#pragma unroll
      for (int c = 0; c < CG; ++c) {
        const float d = f16f(raw[c][23]);
#pragma unroll
        for (int t = 0; t < 4; ++t)
#pragma unroll
          for (int q = 0; q < 4; ++q) acc[c][t][q] = fmaf(d, P[c][t][q], acc[c][t][q]);
      }
    } else {  // Q8_0: one block per 32-value sub-block, its product folded with its own d
#pragma unroll
      for (int b = 0; b < 8; ++b) {
        half8v bf[CG];
        float d[CG];
#pragma unroll
        for (int c = 0; c < CG; ++c) {
          const uint32_t* R = raw[c] + 4 * b;
          const uint32_t q0 = (b & 1) ? R[0] : __builtin_amdgcn_alignbyte(R[1], R[0], 2);
          const uint32_t q1 = (b & 1) ? R[1] : __builtin_amdgcn_alignbyte(R[2], R[1], 2);
          bf[c] = b_codes<0xFFu>(q0 ^ 0x80808080u, q1 ^ 0x80808080u, (_Float16)128);  // q, exact
          d[c] = f16f(R[3]);
        }
#pragma unroll
        for (int t = 0; t < 4; ++t) {
          const half8v af = afrag(b, t);
#pragma unroll
          for (int c = 0; c < CG; ++c) {
            const float4v P = __builtin_amdgcn_mfma_f32_16x16x32_f16(af, bf[c], (float4v){0.f, 0.f, 0.f, 0.f}, 0, 0, 0);
#pragma unroll
            for (int q = 0; q < 4; ++q) acc[c][t][q] = fmaf(d[c], P[q], acc[c][t][q]);
          }
        }
      }
    }
  }
  if (part) {  // a K-slice: raw sums of every staged row, reduced by reduce_kernel
#pragma unroll
    for (int c = 0; c < CG; ++c) {
      if (ncol[c] >= N) continue;
#pragma unroll
      for (int t = 0; t < 4; ++t)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int row = m0 + 16 * t + 4 * kb + r;
          if (row < Mx) part[((size_t)kz * Mx + row) * N + ncol[c]] = acc[c][t][r];
        }
    }
    return;
  }
#pragma unroll
  for (int c = 0; c < CG; ++c) {
    if (ncol[c] >= N) continue;
#pragma unroll
    for (int t = 0; t < 4; ++t)
#pragma unroll
      for (int r = 0; r < 4; r += PAIR ? 2 : 1) {
        const int row = m0 + 16 * t + 4 * kb + r;
        if (row >= Mx) continue;
        float v = acc[c][t][r];
        if constexpr (PAIR) v = (v + acc[c][t][r + 1]) * ldexpf(1.f, -row_exp(rmax[row >> 1]));
        y[(size_t)(PAIR ? row >> 1 : row) * N + ncol[c]] = from_f32<OT>(bias ? v + bias[ncol[c]] : v);
      }
  }
}


// y[m][n] from the K-slices of a split product: the slices' sums in slice order (fp32 rows: the
// hi row's sum plus the lo row's, times 2^-s(m)), + bias[n], as OT. One thread per output.
template <typename OT, bool PAIR>
__global__ __launch_bounds__(256) void reduce_kernel(const float* __restrict__ part, OT* __restrict__ y,
                                                     const float* __restrict__ bias, const float* __restrict__ rmax,
                                                     int M, int N, int ksplit) {
  const size_t i = (size_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= (size_t)M * N) return;
  const int m = (int)(i / N), n = (int)(i % N);
  const size_t Mx = (size_t)M * (PAIR ? 2 : 1), slice = Mx * N;
  const size_t r0 = (size_t)(PAIR ? 2 * m : m) * N + n;
  float v = 0.f;
#pragma unroll 8
  for (int z = 0; z < ksplit; ++z) v += part[z * slice + r0];
  if constexpr (PAIR) {
    float lo = 0.f;
#pragma unroll 8
    for (int z = 0; z < ksplit; ++z) lo += part[z * slice + r0 + N];
    v = (v + lo) * ldexpf(1.f, -row_exp(rmax[m]));
  }
  y[i] = from_f32<OT>(bias ? v + bias[n] : v);
}

// Launch shape: CG column groups per wave, and K split into ksplit slices of ksteps 256-value
// steps when the tile grid alone would leave CUs idle (few rows: the slices' partial sums go
// to the workspace and reduce_kernel adds them in slice order, so results stay deterministic).
struct Plan {
  int cg, mtiles, tiles, ksplit, ksteps;
};
static Plan plan(int M, int K, int N, int x_dtype) {
  const int Mx = (x_dtype == MIQ_F32 ? 2 : 1) * M, nsb = K / 256;
  Plan p;
  p.mtiles = (Mx + kBM - 1) / kBM;
  const long wide = (long)p.mtiles * ((N + 127) / 128);
  p.cg = wide >= 2 * kCUs ? 2 : 1;
  p.tiles = (int)(p.cg == 2 ? wide : (long)p.mtiles * ((N + 63) / 64));
  // split only grids that leave a quarter of the CUs or more idle: at 224 tiles (M = 64 fp16,
  // N = 14336) three slices ran the GEMM no faster (29.7 against 29.1 us: the activation tiles
  // each column tile copies through L2 are the same bytes however K is cut) and added a 5.0 us
  // reduce; at 128 tiles and fewer (the 64-row prefill's q, o, k|v and down) the split won
  p.ksplit = 1;
  if (4 * p.tiles < 3 * kCUs && nsb > 1) p.ksplit = std::min(nsb, (2 * kCUs + p.tiles - 1) / p.tiles);
  p.ksteps = (nsb + p.ksplit - 1) / p.ksplit;
  p.ksplit = (nsb + p.ksteps - 1) / p.ksteps;
  return p;
}

struct Ws {
  size_t xs, rs, rmax, part, bytes;
};
// workspace layout after the shared counter region: staged rows, sub-block sums, row maxima,
// K-slice partial sums
static Ws layout(int M, int K, int N, int x_dtype) {
  const size_t R = x_dtype == MIQ_F32 ? 2 : 1, Mx = R * (size_t)M;
  auto up = [](size_t b) { return (b + 255) & ~(size_t)255; };
  Ws w;
  w.xs = kCounterBytes;
  w.rs = w.xs + up(Mx * K * 2);
  w.rmax = w.rs + up(Mx * (K / 32) * 4);
  w.part = w.rmax + up((size_t)M * 4);
  const Plan p = plan(M, K, N, x_dtype);
  w.bytes = w.part + (p.ksplit > 1 ? up((size_t)p.ksplit * Mx * N * 4) : 0);
  return w;
}

static bool covered(int t) { return t == kQ4_K || t == kQ5_K || t == kQ6_K || t == kQ8_0; }

// The GEMM of type T over staged rows. Two 16-column groups per wave (each activation operand
// read feeds two MFMAs) when that grid still gives every CU two workgroups; otherwise one
// (measured for Q4_K at 4096 -> 14336: fp32 rows at M = 512 288 -> 250 us, fp16 152 -> 149 us;
// at M = 64 the halved grid was slower, 36 -> 51 us), and K split when even that grid is small.
template <int T>
static int gemm_t(const __half* xs, const float* rs, const float* rmax, float* part, const uint8_t* w,
                  const float* bias, void* out, int out_dtype, int M, int x_dtype, int K, int N, hipStream_t st) {
  const int R = x_dtype == MIQ_F32 ? 2 : 1, Mx = R * M;
  const Plan pl = plan(M, K, N, x_dtype);
  const dim3 grid((unsigned)(pl.tiles * pl.ksplit));
  float* pp = pl.ksplit > 1 ? part : nullptr;
  auto go = [&](auto* dst, auto pair) {
    using OT = std::remove_pointer_t<decltype(dst)>;
    constexpr bool P = decltype(pair)::value;
    if (pl.cg == 2)
      hipLaunchKernelGGL((gemm_kernel<T, 2, OT, P>), grid, dim3(256), 0, st, xs, rs, w, dst, bias, rmax, Mx, K, N,
                         pl.mtiles, pl.tiles, pl.ksteps, pp);
    else
      hipLaunchKernelGGL((gemm_kernel<T, 1, OT, P>), grid, dim3(256), 0, st, xs, rs, w, dst, bias, rmax, Mx, K, N,
                         pl.mtiles, pl.tiles, pl.ksteps, pp);
    int rc = check_launch("ggml_gemm");
    if (rc || !pp) return rc;
    const size_t n = (size_t)M * N;
    hipLaunchKernelGGL((reduce_kernel<OT, P>), dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st, pp, dst, bias,
                       rmax, M, N, pl.ksplit);
    return check_launch("ggml_gemm reduce");
  };
  if (R == 1) {
    if (out_dtype == MIQ_F16) return go(static_cast<__half*>(out), std::false_type{});
    return go(static_cast<float*>(out), std::false_type{});
  }
  if (out_dtype == MIQ_F16) return go(static_cast<__half*>(out), std::true_type{});
  return go(static_cast<float*>(out), std::true_type{});
}

}  // namespace kg
}  // namespace miq

using namespace miq;

extern "C" int miq_ggml_gemm_workspace(int M, int K, int N, int x_dtype, int ggml_type, size_t* bytes) {
  MIQ_REQUIRE(bytes, MIQ_ERR_INVALID, "ggml_gemm_workspace: null output");
  MIQ_REQUIRE(kg::covered(ggml_type), MIQ_ERR_UNSUPPORTED, "ggml_gemm_workspace: ggml type %d has no GEMM",
              ggml_type);
  MIQ_REQUIRE(M >= 0 && K > 0 && N > 0 && K % 256 == 0, MIQ_ERR_INVALID, "ggml_gemm_workspace: M=%d K=%d N=%d", M, K,
              N);
  MIQ_REQUIRE(x_dtype == MIQ_F16 || x_dtype == MIQ_F32, MIQ_ERR_UNSUPPORTED, "ggml_gemm_workspace: x dtype");
  *bytes = M == 0 ? 0 : kg::layout(M, K, N, x_dtype).bytes;
  return MIQ_OK;
}

extern "C" int miq_ggml_gemm(const void* x, int x_dtype, const uint8_t* w, int ggml_type, const float* bias, void* out,
                             int out_dtype, int M, int K, int N, void* workspace, size_t ws_bytes, void* stream) {
  MIQ_REQUIRE(kg::covered(ggml_type), MIQ_ERR_UNSUPPORTED, "ggml_gemm: ggml type %d has no GEMM", ggml_type);
  MIQ_REQUIRE(M >= 0 && K > 0 && N > 0, MIQ_ERR_INVALID, "ggml_gemm: M=%d K=%d N=%d", M, K, N);
  MIQ_REQUIRE(K % 256 == 0, MIQ_ERR_INVALID, "ggml_gemm: K=%d is not a multiple of 256", K);
  MIQ_REQUIRE(x_dtype == MIQ_F16 || x_dtype == MIQ_F32, MIQ_ERR_UNSUPPORTED, "ggml_gemm: x dtype");
  MIQ_REQUIRE(out_dtype == MIQ_F16 || out_dtype == MIQ_F32, MIQ_ERR_UNSUPPORTED, "ggml_gemm: out dtype");
  if (M == 0) return MIQ_OK;
  MIQ_REQUIRE(x && w && out && workspace, MIQ_ERR_INVALID, "ggml_gemm: null pointer");
  MIQ_REQUIRE(aligned(w, 16) && aligned(x, 16) && aligned(workspace, 256), MIQ_ERR_ALIGN,
              "ggml_gemm: x and weight 16-byte, workspace 256-byte aligned");
  const kg::Ws L = kg::layout(M, K, N, x_dtype);
  MIQ_REQUIRE(ws_bytes >= L.bytes, MIQ_ERR_INVALID, "ggml_gemm: workspace %zu bytes, need %zu", ws_bytes, L.bytes);
  MIQ_REQUIRE(K <= 16384, MIQ_ERR_UNSUPPORTED, "ggml_gemm: K=%d too large to stage", K);
  hipStream_t st = static_cast<hipStream_t>(stream);
  unsigned char* b = static_cast<unsigned char*>(workspace);
  __half* xs = reinterpret_cast<__half*>(b + L.xs);
  float* rs = reinterpret_cast<float*>(b + L.rs);
  float* rmax = reinterpret_cast<float*>(b + L.rmax);
  float* part = reinterpret_cast<float*>(b + L.part);
  if (x_dtype == MIQ_F32) {
    if ((size_t)K * 4 > 64 * 1024) {
      const int rc = require_lds("ggml_gemm staging", (size_t)K * 4);
      if (rc) return rc;
    }
    hipLaunchKernelGGL(kg::stage_kernel<float>, dim3(M), dim3(256), (size_t)K * 4, st, static_cast<const float*>(x), xs,
                       rs, rmax, K);
  } else {
    hipLaunchKernelGGL(kg::stage_kernel<__half>, dim3(M), dim3(256), 0, st, static_cast<const __half*>(x), xs, rs, rmax,
                       K);
  }
  const int rc = check_launch("ggml_gemm staging");
  if (rc) return rc;
  switch (ggml_type) {
    case kg::kQ4_K: return kg::gemm_t<kg::kQ4_K>(xs, rs, rmax, part, w, bias, out, out_dtype, M, x_dtype, K, N, st);
    case kg::kQ5_K: return kg::gemm_t<kg::kQ5_K>(xs, rs, rmax, part, w, bias, out, out_dtype, M, x_dtype, K, N, st);
    case kg::kQ6_K: return kg::gemm_t<kg::kQ6_K>(xs, rs, rmax, part, w, bias, out, out_dtype, M, x_dtype, K, N, st);
    default: return kg::gemm_t<kg::kQ8_0>(xs, rs, rmax, part, w, bias, out, out_dtype, M, x_dtype, K, N, st);
  }
}

extern "C" int miq_q4k_gemm_workspace(int M, int K, int N, int x_dtype, size_t* bytes) {
  return miq_ggml_gemm_workspace(M, K, N, x_dtype, kg::kQ4_K, bytes);
}

extern "C" int miq_q4k_gemm(const void* x, int x_dtype, const uint8_t* w, const float* bias, void* out, int out_dtype,
                            int M, int K, int N, void* workspace, size_t ws_bytes, void* stream) {
  return miq_ggml_gemm(x, x_dtype, w, kg::kQ4_K, bias, out, out_dtype, M, K, N, workspace, ws_bytes, stream);
}
