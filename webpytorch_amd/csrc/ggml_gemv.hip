// The GGUF block types beside Q4_K: decode GEMV and fp32 dequant over the blocks as the file
// stores them (gfx950). Q8_0 and Q6_K (the rest of a Q4_K_M file) are laid out below; Q4_0,
// Q4_1, Q5_0, Q5_1, IQ4_NL (32-value blocks), IQ4_XS, Q5_K, Q2_K and Q3_K (256-value
// super-blocks) follow llama.cpp's published block layouts, each given beside its decoder.
//
// Q8_0 block (32 weights, 34 bytes): fp16 d at 0, 32 int8 codes at 2; weight i = d * q[i].
// Q6_K super-block (256 weights, 210 bytes): ql[128] at 0 (low 4 bits), qh[64] at 128 (high 2
// bits), 16 int8 scales at 192, fp16 d at 208. Half h (128 weights) uses ql[64h..], qh[32h..],
// scales[8h..]; weight 128h + 32j + l (j < 4, l < 32) has code
//   c = ((ql[64h + l + 32 (j & 1)] >> 4 (j >> 1)) & 15) | (((qh[32h + l] >> 2j) & 3) << 4)
// and value d * scales[8h + l / 16 + 2j] * (c - 32).
// A weight matrix is N rows of K / (values per block) consecutive blocks, as the file holds it.
//
// Neither block size is a multiple of four, so block starts are only 2-byte aligned. Every
// load here is 4-byte aligned (a dword at a rounded-down address, the wanted bytes shifted out
// with v_alignbyte), 2-byte (fp16 d) or 1-byte (a Q6_K scale), and no load reaches past the
// last byte of the block it serves (bytes before the block, at most 2, belong to the previous
// block or the row before).
//
// Mapping: a workgroup stages one activation row in LDS (fp32) with sums over each lane's run
// of activations; each wave takes R = 4 output rows at a time; lanes split the blocks of a row
// (Q8_0: 4 lanes per block, 8 weights each; Q6_K: 16 lanes per super-block, the 16 weights of
// one scale each), unpack codes into bytes and convert them with v_cvt_f32_ubyte*; a lane's
// partial is scale * (sum x * (q + offset) - offset * sum x) with the offset that makes codes
// unsigned (128 for Q8_0, 32 for Q6_K).
#include <type_traits>

#include "miq_common.h"
#include "iq_grids.h"
#include "moe_route.h"

namespace miq {
namespace gg {

// ggml type ids
constexpr int kQ4_0 = 2, kQ4_1 = 3, kQ5_0 = 6, kQ5_1 = 7, kQ8_0 = 8, kQ2_K = 10, kQ3_K = 11, kQ5_K = 13, kQ6_K = 14,
              kIQ4_NL = 20, kIQ4_XS = 23;
// the codebook-grid i-quants, ternary, fp4 and 1/2-bit types (lanes take consecutive values)
constexpr int kIQ2_XXS = 16, kIQ2_XS = 17, kIQ3_XXS = 18, kIQ1_S = 19, kIQ3_S = 21, kIQ2_S = 22, kIQ1_M = 29,
              kTQ1_0 = 34, kTQ2_0 = 35, kMXFP4 = 39, kNVFP4 = 40, kQ1_0 = 41, kQ2_0 = 42;
// unquantized 2-D weights (one value per "block"): their own kernel below
constexpr int kF32 = 0, kF16 = 1, kBF16 = 30;

// Values and bytes per block; lanes per block and values per lane of the GEMV; rows a wave
// walks (the fastest of 1, 2 and 4 per type at 4096 -> 14336).
template <int T> struct Blk;
template <> struct Blk<kQ8_0> { static constexpr int VALS = 32, BYTES = 34, LPB = 4, VPL = 8, ROWS = 2; };
template <> struct Blk<kQ6_K> { static constexpr int VALS = 256, BYTES = 210, LPB = 16, VPL = 16, ROWS = 1; };
template <> struct Blk<kQ4_0> { static constexpr int VALS = 32, BYTES = 18, LPB = 4, VPL = 8, ROWS = 4; };
template <> struct Blk<kQ4_1> { static constexpr int VALS = 32, BYTES = 20, LPB = 4, VPL = 8, ROWS = 2; };
template <> struct Blk<kQ5_0> { static constexpr int VALS = 32, BYTES = 22, LPB = 4, VPL = 8, ROWS = 2; };
template <> struct Blk<kQ5_1> { static constexpr int VALS = 32, BYTES = 24, LPB = 4, VPL = 8, ROWS = 4; };
template <> struct Blk<kIQ4_NL> { static constexpr int VALS = 32, BYTES = 18, LPB = 4, VPL = 8, ROWS = 2; };
template <> struct Blk<kIQ4_XS> { static constexpr int VALS = 256, BYTES = 136, LPB = 16, VPL = 16, ROWS = 2; };
template <> struct Blk<kQ5_K> { static constexpr int VALS = 256, BYTES = 176, LPB = 16, VPL = 16, ROWS = 1; };
template <> struct Blk<kQ2_K> { static constexpr int VALS = 256, BYTES = 84, LPB = 16, VPL = 16, ROWS = 2; };
template <> struct Blk<kQ3_K> { static constexpr int VALS = 256, BYTES = 110, LPB = 16, VPL = 16, ROWS = 1; };
// Lane t of these takes values VPL t .. VPL t + VPL - 1 of its block (SEQ).
template <> struct Blk<kIQ2_XXS> { static constexpr int VALS = 256, BYTES = 66, LPB = 16, VPL = 16, ROWS = 2, SEQ = 1; };
template <> struct Blk<kIQ2_XS> { static constexpr int VALS = 256, BYTES = 74, LPB = 16, VPL = 16, ROWS = 2, SEQ = 1; };
template <> struct Blk<kIQ2_S> { static constexpr int VALS = 256, BYTES = 82, LPB = 16, VPL = 16, ROWS = 2, SEQ = 1; };
template <> struct Blk<kIQ3_XXS> { static constexpr int VALS = 256, BYTES = 98, LPB = 16, VPL = 16, ROWS = 2, SEQ = 1; };
template <> struct Blk<kIQ3_S> { static constexpr int VALS = 256, BYTES = 110, LPB = 16, VPL = 16, ROWS = 2, SEQ = 1; };
template <> struct Blk<kIQ1_S> { static constexpr int VALS = 256, BYTES = 50, LPB = 16, VPL = 16, ROWS = 2, SEQ = 1; };
template <> struct Blk<kIQ1_M> { static constexpr int VALS = 256, BYTES = 56, LPB = 16, VPL = 16, ROWS = 2, SEQ = 1; };
template <> struct Blk<kTQ1_0> { static constexpr int VALS = 256, BYTES = 54, LPB = 16, VPL = 16, ROWS = 2, SEQ = 1; };
template <> struct Blk<kTQ2_0> { static constexpr int VALS = 256, BYTES = 66, LPB = 16, VPL = 16, ROWS = 2, SEQ = 1; };
template <> struct Blk<kMXFP4> { static constexpr int VALS = 32, BYTES = 17, LPB = 4, VPL = 8, ROWS = 2, SEQ = 1; };
template <> struct Blk<kNVFP4> { static constexpr int VALS = 64, BYTES = 36, LPB = 8, VPL = 8, ROWS = 2, SEQ = 1; };
template <> struct Blk<kQ1_0> { static constexpr int VALS = 128, BYTES = 18, LPB = 16, VPL = 8, ROWS = 2, SEQ = 1; };
template <> struct Blk<kQ2_0> { static constexpr int VALS = 64, BYTES = 18, LPB = 8, VPL = 8, ROWS = 2, SEQ = 1; };
// Q4_K in the generic template: the grouped expert GEMV (miq_q4k_gemv is the dense one)
constexpr int kQ4_K = 12;
template <> struct Blk<kQ4_K> { static constexpr int VALS = 256, BYTES = 144, LPB = 16, VPL = 16, ROWS = 2, SEQ = 1; };
template <int T, typename = void> struct SeqLanes { static constexpr bool value = false; };
template <int T> struct SeqLanes<T, std::void_t<decltype(Blk<T>::SEQ)>> { static constexpr bool value = true; };

__device__ __forceinline__ uint32_t ld32(const uint8_t* w, size_t a) {
  return *reinterpret_cast<const uint32_t*>(w + a);  // a % 4 == 0
}
__device__ __forceinline__ uint32_t ld16(const uint8_t* w, size_t a) {
  return *reinterpret_cast<const unsigned short*>(w + a);  // a % 2 == 0
}
__device__ __forceinline__ float f16_at(const uint8_t* w, size_t a) {
  return __half2float(__ushort_as_half((unsigned short)ld16(w, a)));
}
// the four unsigned bytes of c against x[0..3] (each conversion is one v_cvt_f32_ubyteN)
__device__ __forceinline__ float dot4u(uint32_t c, const float* x, float p) {
  p = fmaf(x[0], (float)(c & 0xFFu), p);
  p = fmaf(x[1], (float)((c >> 8) & 0xFFu), p);
  p = fmaf(x[2], (float)((c >> 16) & 0xFFu), p);
  return fmaf(x[3], (float)(c >> 24), p);
}

// Position of lane t's first weight within its block. 32-value types: lane t takes the low
// (t < 2) or high nibbles of 8 code bytes, i.e. values 16 (t >> 1) + 8 (t & 1) .. + 7. Q2_K /
// Q3_K (and Q6_K): lane t = (h, j, u) takes the 16 values 128 h + 32 j + 16 u.. of one scale.
// Q5_K: lane t = (g, hi, part) takes values 64 g + 32 hi + 16 part... IQ4_XS: lane t = (ib, hi)
// takes values 32 ib + 16 hi...
template <int T> __device__ __forceinline__ int lane_k(int t) {
  if constexpr (SeqLanes<T>::value) return Blk<T>::VPL * t;
  else if constexpr (T == kQ8_0) return 8 * t;
  else if constexpr (Blk<T>::VALS == 32) return 16 * (t >> 1) + 8 * (t & 1);
  else if constexpr (T == kQ5_K) return 64 * (t >> 2) + 32 * ((t >> 1) & 1) + 16 * (t & 1);
  else if constexpr (T == kIQ4_XS) return 32 * (t >> 1) + 16 * (t & 1);
  else return 128 * (t >> 3) + 32 * ((t >> 1) & 3) + 16 * (t & 1);
}

// Four bytes at a 2-byte-aligned address (two 2-byte loads: no read leaves the block).
__device__ __forceinline__ uint32_t u32_at2(const uint8_t* w, size_t a) { return ld16(w, a) | (ld16(w, a + 2) << 16); }
// 4 codes of a 4-bit codebook (IQ4_NL / IQ4_XS) as unsigned bytes kv + 128, from 4 nibble bytes
// (0..15) in c: two byte selects over the 16-entry table and a pick by bit 3.
__device__ __forceinline__ uint32_t iq4_lookup(uint32_t c) {
  const uint32_t sel = c & 0x07070707u;
  const uint32_t a = __builtin_amdgcn_perm(0x766A5D4Fu, 0x3F2D1801u, sel);  // kv[0..7] + 128
  const uint32_t b = __builtin_amdgcn_perm(0xF1D9C5B5u, 0xA6998D81u, sel);  // kv[8..15] + 128
  const uint32_t m = ((c >> 3) & 0x01010101u) * 0xFFu;
  return (a & ~m) | (b & m);
}
// bits [sh, sh + 4) of qbits as 16 in bytes 0..3 (a 5-bit code's fifth bit)
__device__ __forceinline__ uint32_t fifth4(uint32_t qbits, int sh) {
  const uint32_t b = qbits >> sh;
  return (((b & 1u) | ((b & 2u) << 7) | ((b & 4u) << 14) | ((b & 8u) << 21))) << 4;
}

// Lane t's share of one block at byte offset bs: its partial of sum_k x[k] * w[k], given its
// activations x (VPL values from lane_k) and their sum xs.
template <int T> __device__ __forceinline__ float lane_dot(const uint8_t* w, size_t bs, int t, const float* x, float xs);

template <> __device__ __forceinline__ float lane_dot<kQ8_0>(const uint8_t* w, size_t bs, int t, const float* x,
                                                             float xs) {
  // codes [a, a + 8): with s = a % 4 (0 or 2), dwords at a - s and a - s + 4, and the last two
  // bytes from a 2-byte load at a + 6 (a + 8 is at most the block's end)
  const size_t a = bs + 2 + 8 * t;
  const uint32_t s = (uint32_t)(a & 3);
  const uint32_t d0 = ld32(w, a - s), d1 = ld32(w, a - s + 4), u = ld16(w, a + 6);
  const uint32_t w0 = __builtin_amdgcn_alignbyte(d1, d0, s);
  const uint32_t w1 = s ? __builtin_amdgcn_alignbyte(u, d1, 2) : d1;
  float p = dot4u(w0 ^ 0x80808080u, x, 0.f);  // q + 128
  p = dot4u(w1 ^ 0x80808080u, x + 4, p);
  return f16_at(w, bs) * fmaf(-128.f, xs, p);
}

template <> __device__ __forceinline__ float lane_dot<kQ6_K>(const uint8_t* w, size_t bs, int t, const float* x,
                                                             float xs) {
  const int h = t >> 3, j = (t >> 1) & 3, e = t & 1;
  // 16 ql bytes at aql and 16 qh bytes at aqh (same residue mod 4): five dwords from a - s each;
  // the last ends at most 20 bytes past a, inside the block (a + 20 <= bs + 196)
  const size_t aql = bs + 64 * h + 32 * (j & 1) + 16 * e, aqh = bs + 128 + 32 * h + 16 * e;
  const uint32_t s = (uint32_t)(aql & 3);
  uint32_t L[5], Hq[5];
#pragma unroll
  for (int i = 0; i < 5; ++i) {
    L[i] = ld32(w, aql - s + 4 * i);
    Hq[i] = ld32(w, aqh - s + 4 * i);
  }
  const int8_t sc = (int8_t)w[bs + 192 + 8 * h + e + 2 * j];
  const float d = f16_at(w, bs + 208);
  const uint32_t nib = 4 * (j >> 1), hs = 2 * j;
  float p = 0.f;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const uint32_t ql = __builtin_amdgcn_alignbyte(L[i + 1], L[i], s);
    const uint32_t qh = __builtin_amdgcn_alignbyte(Hq[i + 1], Hq[i], s);
    const uint32_t c = ((ql >> nib) & 0x0F0F0F0Fu) | (((qh >> hs) & 0x03030303u) << 4);
    p = dot4u(c, x + 4 * i, p);
  }
  return (d * (float)sc) * fmaf(-32.f, xs, p);
}

// The 32-value types. Q4_0 (18 bytes): fp16 d, 16 code bytes; d (q - 8). Q4_1 (20): fp16 d,
// fp16 m, 16 code bytes; d q + m. Q5_0 (22): fp16 d, u32 fifth bits, 16 code bytes; d (q - 16).
// Q5_1 (24): fp16 d, fp16 m, u32 fifth bits, 16 code bytes; d q + m. IQ4_NL (18): fp16 d, 16 code
// bytes; d kv[q] over the 16-entry codebook. Value j < 16 is the low nibble of code byte j and
// value 16 + j the high one; a 5-bit code takes bit j (or j + 16) of the fifth-bit word.
// Lane t's 8 code bytes (nibble t >> 1) dotted with x.
template <int T> __device__ __forceinline__ float lane_dot32(const uint8_t* w, size_t bs, int t, const float* x,
                                                            float xs) {
  constexpr int QS = T == kQ4_0 || T == kIQ4_NL ? 2 : T == kQ4_1 ? 4 : T == kQ5_0 ? 6 : 8;
  const int j0 = 8 * (t & 1), hi = t >> 1;
  const uint32_t c0 = (u32_at2(w, bs + QS + j0) >> (4 * hi)) & 0x0F0F0F0Fu;
  const uint32_t c1 = (u32_at2(w, bs + QS + j0 + 4) >> (4 * hi)) & 0x0F0F0F0Fu;
  const float d = f16_at(w, bs);
  if constexpr (T == kIQ4_NL) {
    const float p = dot4u(iq4_lookup(c1), x + 4, dot4u(iq4_lookup(c0), x, 0.f));  // sum x (kv + 128)
    return d * fmaf(-128.f, xs, p);
  } else if constexpr (T == kQ4_0 || T == kQ4_1) {
    const float p = dot4u(c1, x + 4, dot4u(c0, x, 0.f));
    if constexpr (T == kQ4_0) return d * fmaf(-8.f, xs, p);
    else return fmaf(d, p, f16_at(w, bs + 2) * xs);
  } else {  // Q5_0 / Q5_1: the fifth bit of value j (of 16) in nibble half hi is bit j + 16 hi of qh
    const uint32_t qh = u32_at2(w, bs + (T == kQ5_0 ? 2 : 4));
    const int sh = j0 + 16 * hi;
    const float p = dot4u(c1 | fifth4(qh, sh + 4), x + 4, dot4u(c0 | fifth4(qh, sh), x, 0.f));
    if constexpr (T == kQ5_0) return d * fmaf(-16.f, xs, p);
    else return fmaf(d, p, f16_at(w, bs + 2) * xs);
  }
}
template <> __device__ __forceinline__ float lane_dot<kQ4_0>(const uint8_t* w, size_t bs, int t, const float* x, float xs) { return lane_dot32<kQ4_0>(w, bs, t, x, xs); }
template <> __device__ __forceinline__ float lane_dot<kQ4_1>(const uint8_t* w, size_t bs, int t, const float* x, float xs) { return lane_dot32<kQ4_1>(w, bs, t, x, xs); }
template <> __device__ __forceinline__ float lane_dot<kQ5_0>(const uint8_t* w, size_t bs, int t, const float* x, float xs) { return lane_dot32<kQ5_0>(w, bs, t, x, xs); }
template <> __device__ __forceinline__ float lane_dot<kQ5_1>(const uint8_t* w, size_t bs, int t, const float* x, float xs) { return lane_dot32<kQ5_1>(w, bs, t, x, xs); }
template <> __device__ __forceinline__ float lane_dot<kIQ4_NL>(const uint8_t* w, size_t bs, int t, const float* x, float xs) { return lane_dot32<kIQ4_NL>(w, bs, t, x, xs); }

// 16 code bytes at a 2-byte-aligned address, as four words.
__device__ __forceinline__ void load16(const uint8_t* w, size_t a, uint32_t* c) {
#pragma unroll
  for (int i = 0; i < 4; ++i) c[i] = u32_at2(w, a + 4 * i);
}

// IQ4_XS (256 values, 136 bytes): fp16 d, u16 high scale bits, 4 bytes of low scale nibbles,
// 128 code bytes; sub-block ib (32 values, codes as IQ4_NL in bytes 8 + 16 ib..) has
// ls = nibble ib of the low bytes | bits 2 ib, 2 ib + 1 of the u16 << 4 and value d (ls - 32) kv[q].
template <> __device__ __forceinline__ float lane_dot<kIQ4_XS>(const uint8_t* w, size_t bs, int t, const float* x,
                                                               float xs) {
  const int ib = t >> 1, hi = t & 1;
  uint32_t c[4];
  load16(w, bs + 8 + 16 * ib, c);
  float p = 0.f;
#pragma unroll
  for (int i = 0; i < 4; ++i) p = dot4u(iq4_lookup((c[i] >> (4 * hi)) & 0x0F0F0F0Fu), x + 4 * i, p);
  const int ls = ((w[bs + 4 + ib / 2] >> (4 * (ib & 1))) & 15) | (((int)(ld16(w, bs + 2) >> (2 * ib)) & 3) << 4);
  return (f16_at(w, bs) * (float)(ls - 32)) * fmaf(-128.f, xs, p);
}

// The Q4_K / Q5_K 6-bit scale and min of sub-block j from the 12 packed bytes at a.
__device__ __forceinline__ void scale_min_k4(const uint8_t* w, size_t a, int j, int* sc, int* mn) {
  if (j < 4) {
    *sc = w[a + j] & 63;
    *mn = w[a + j + 4] & 63;
  } else {
    *sc = (w[a + j + 4] & 15) | ((w[a + j - 4] >> 6) << 4);
    *mn = (w[a + j + 4] >> 4) | ((w[a + j] >> 6) << 4);
  }
}

// Q5_K (256 values, 176 bytes): fp16 d, fp16 dmin, 12 bytes of 6-bit scales/mins, qh[32],
// qs[128]. Sub-block 2g + hi (32 values) takes nibble hi of qs[32 g + l] plus 16 times bit
// 2g + hi of qh[l]; value (d sc) q - dmin m.
template <> __device__ __forceinline__ float lane_dot<kQ5_K>(const uint8_t* w, size_t bs, int t, const float* x,
                                                             float xs) {
  const int g = t >> 2, hi = (t >> 1) & 1, part = t & 1, sb = 2 * g + hi;
  uint32_t c[4], h[4];
  load16(w, bs + 48 + 32 * g + 16 * part, c);
  load16(w, bs + 16 + 16 * part, h);
  float p = 0.f;
#pragma unroll
  for (int i = 0; i < 4; ++i)
    p = dot4u(((c[i] >> (4 * hi)) & 0x0F0F0F0Fu) | (((h[i] >> sb) & 0x01010101u) << 4), x + 4 * i, p);
  int sc, mn;
  scale_min_k4(w, bs + 4, sb, &sc, &mn);
  return (f16_at(w, bs) * (float)sc) * p - (f16_at(w, bs + 2) * (float)mn) * xs;
}

// Q2_K (256 values, 84 bytes): 16 scale bytes (low nibble scale, high nibble min), qs[64],
// fp16 d, fp16 dmin. Value 128 h + 32 j + 16 u + l is bits 2j, 2j + 1 of qs[32 h + 16 u + l]
// with scale byte 8 h + 2 j + u; value (d sc) q - dmin m.
template <> __device__ __forceinline__ float lane_dot<kQ2_K>(const uint8_t* w, size_t bs, int t, const float* x,
                                                             float xs) {
  const int h = t >> 3, j = (t >> 1) & 3, u = t & 1;
  uint32_t c[4];
  load16(w, bs + 16 + 32 * h + 16 * u, c);
  float p = 0.f;
#pragma unroll
  for (int i = 0; i < 4; ++i) p = dot4u((c[i] >> (2 * j)) & 0x03030303u, x + 4 * i, p);
  const int sc = w[bs + 8 * h + 2 * j + u];
  return (f16_at(w, bs + 80) * (float)(sc & 15)) * p - (f16_at(w, bs + 82) * (float)(sc >> 4)) * xs;
}

// Q3_K (256 values, 110 bytes): hmask[32], qs[64], 12 bytes of 6-bit scales, fp16 d. Value
// 128 h + 32 j + 16 u + l is bits 2j of qs[32 + 32 h + 16 u + l], minus 4 unless bit 4 h + j of
// hmask[16 u + l] is set; scale i = 8 h + 2 j + u has nibble i / 8 of byte i % 8 and bit pair
// i / 4 of byte 8 + i % 4 as its high bits, minus 32; value d scale q.
template <> __device__ __forceinline__ float lane_dot<kQ3_K>(const uint8_t* w, size_t bs, int t, const float* x,
                                                             float xs) {
  const int h = t >> 3, j = (t >> 1) & 3, u = t & 1, is = 8 * h + 2 * j + u;
  uint32_t c[4], m[4];
  load16(w, bs + 32 + 32 * h + 16 * u, c);
  load16(w, bs + 16 * u, m);
  float p = 0.f;  // sum x (v + 4), v + 4 = 2-bit code + 4 * (hmask bit)
#pragma unroll
  for (int i = 0; i < 4; ++i)
    p = dot4u(((c[i] >> (2 * j)) & 0x03030303u) | (((m[i] >> (4 * h + j)) & 0x01010101u) << 2), x + 4 * i, p);
  const int sc = (((int)w[bs + 96 + (is & 7)] >> (4 * (is >> 3))) & 15) |
                 ((((int)w[bs + 104 + (is & 3)] >> (2 * (is >> 2))) & 3) << 4);
  return (f16_at(w, bs + 108) * (float)(sc - 32)) * fmaf(-4.f, xs, p);
}

// Q4_K (144 bytes): fp16 d, fp16 dmin, 12 bytes of 6-bit scales/mins, qs[128]; sub-block sb
// (32 values) takes nibble sb % 2 of qs[32 (sb / 2) + l]; value (d sc) q - dmin m. Lane t takes
// half t % 2 of sub-block t / 2.
template <> __device__ __forceinline__ float lane_dot<kQ4_K>(const uint8_t* w, size_t bs, int t, const float* x,
                                                             float xs) {
  const int sb = t >> 1, half = t & 1;
  uint32_t c[4];
  load16(w, bs + 16 + 32 * (sb >> 1) + 16 * half, c);
  float p = 0.f;
#pragma unroll
  for (int i = 0; i < 4; ++i) p = dot4u((c[i] >> (4 * (sb & 1))) & 0x0F0F0F0Fu, x + 4 * i, p);
  int sc, mn;
  scale_min_k4(w, bs + 4, sb, &sc, &mn);
  return (f16_at(w, bs) * (float)sc) * p - (f16_at(w, bs + 2) * (float)mn) * xs;
}

// ---- the codebook-grid i-quants (llama.cpp's dequantize_row_iq*) ----------------------------
// A 256-value super-block holds 8 sub-blocks of 32 values, each 4 groups of 8 values; a group is
// one (IQ2) or two (IQ3) codebook entries with a sign mask (bit j negates value j). Lane t takes
// sub-block ib = t / 2, groups 2 h and 2 h + 1 (h = t % 2). The signs of IQ2_XXS / IQ2_XS /
// IQ3_XXS are 7-bit indices whose eighth bit is their parity; IQ2_S / IQ3_S store the byte.
__device__ __forceinline__ uint32_t ksign(uint32_t s) { return s | ((uint32_t)(__builtin_popcount(s) & 1) << 7); }
// x with its sign flipped where bit j of m is set
__device__ __forceinline__ float sgn(float x, uint32_t m, int j) {
  return __int_as_float(__float_as_int(x) ^ (int)(((m >> j) & 1u) << 31));
}
// the 8 unsigned bytes of g (value j in byte j) against x[0..7], signs from m
__device__ __forceinline__ float dot8s(uint64_t g, uint32_t m, const float* x, float p) {
  const uint32_t lo = (uint32_t)g, hi = (uint32_t)(g >> 32);
#pragma unroll
  for (int j = 0; j < 4; ++j) p = fmaf(sgn(x[j], m, j), (float)((lo >> (8 * j)) & 0xFFu), p);
#pragma unroll
  for (int j = 0; j < 4; ++j) p = fmaf(sgn(x[4 + j], m, 4 + j), (float)((hi >> (8 * j)) & 0xFFu), p);
  return p;
}
__device__ __forceinline__ uint64_t iq3_pair(uint32_t i1, uint32_t i2) {
  return (uint64_t)iq::kIQ3XXS[i1] | ((uint64_t)iq::kIQ3XXS[i2] << 32);
}
__device__ __forceinline__ uint64_t iq3s_pair(uint32_t i1, uint32_t i2) {
  return (uint64_t)iq::kIQ3S[i1] | ((uint64_t)iq::kIQ3S[i2] << 32);
}

// IQ2_XXS (66 bytes): fp16 d, then per sub-block two words: a0 = four grid indices (bytes),
// a1 = four 7-bit sign indices (bits 7 l..) and a 4-bit scale (bits 28-31);
// value (d (0.5 + scale) / 4) * grid * sign.
template <> __device__ __forceinline__ float lane_dot<kIQ2_XXS>(const uint8_t* w, size_t bs, int t, const float* x,
                                                                float) {
  const int ib = t >> 1, h = t & 1;
  const uint32_t a0 = u32_at2(w, bs + 2 + 8 * ib), a1 = u32_at2(w, bs + 6 + 8 * ib);
  float p = 0.f;
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    const int l = 2 * h + i;
    p = dot8s(iq::kIQ2XXS[(a0 >> (8 * l)) & 0xFFu], ksign((a1 >> (7 * l)) & 127u), x + 8 * i, p);
  }
  return (f16_at(w, bs) * (0.5f + (float)(a1 >> 28)) * 0.25f) * p;
}

// IQ2_XS (74 bytes): fp16 d, 32 u16 codes (9-bit grid index, 7-bit sign index), 8 scale bytes
// (low nibble: groups 0-1 of the sub-block, high: groups 2-3).
template <> __device__ __forceinline__ float lane_dot<kIQ2_XS>(const uint8_t* w, size_t bs, int t, const float* x,
                                                               float) {
  const int ib = t >> 1, h = t & 1;
  float p = 0.f;
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    const uint32_t q = ld16(w, bs + 2 + 2 * (4 * ib + 2 * h + i));
    p = dot8s(iq::kIQ2XS[q & 511u], ksign(q >> 9), x + 8 * i, p);
  }
  const uint32_t sc = (w[bs + 66 + ib] >> (4 * h)) & 15u;
  return (f16_at(w, bs) * (0.5f + (float)sc) * 0.25f) * p;
}

// IQ2_S (82 bytes): fp16 d, 32 low index bytes, 32 sign bytes, 8 high-bit bytes (2 bits per
// group), 8 scale bytes as IQ2_XS.
template <> __device__ __forceinline__ float lane_dot<kIQ2_S>(const uint8_t* w, size_t bs, int t, const float* x,
                                                              float) {
  const int ib = t >> 1, h = t & 1;
  const uint32_t qh = w[bs + 66 + ib];
  float p = 0.f;
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    const int l = 2 * h + i;
    const uint32_t idx = w[bs + 2 + 4 * ib + l] | ((qh << (8 - 2 * l)) & 0x300u);
    p = dot8s(iq::kIQ2S[idx], w[bs + 34 + 4 * ib + l], x + 8 * i, p);
  }
  const uint32_t sc = (w[bs + 74 + ib] >> (4 * h)) & 15u;
  return (f16_at(w, bs) * (0.5f + (float)sc) * 0.25f) * p;
}

// IQ3_XXS (98 bytes): fp16 d, 64 grid index bytes (two 4-value entries per group), then one word
// per sub-block: four 7-bit sign indices and a 4-bit scale; value (d (0.5 + scale) / 2) * grid * sign.
template <> __device__ __forceinline__ float lane_dot<kIQ3_XXS>(const uint8_t* w, size_t bs, int t, const float* x,
                                                                float) {
  const int ib = t >> 1, h = t & 1;
  const uint32_t a = u32_at2(w, bs + 66 + 4 * ib);
  float p = 0.f;
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    const int l = 2 * h + i;
    const size_t q = bs + 2 + 8 * ib + 2 * l;
    p = dot8s(iq3_pair(w[q], w[q + 1]), ksign((a >> (7 * l)) & 127u), x + 8 * i, p);
  }
  return (f16_at(w, bs) * (0.5f + (float)(a >> 28)) * 0.5f) * p;
}

// IQ3_S (110 bytes): fp16 d, 64 low index bytes, 8 high-bit bytes (bit 2 l of qh[ib] for entry
// 2 l, bit 2 l + 1 for entry 2 l + 1), 32 sign bytes, 4 scale bytes (a nibble per sub-block);
// value d (1 + 2 scale) * grid * sign.
template <> __device__ __forceinline__ float lane_dot<kIQ3_S>(const uint8_t* w, size_t bs, int t, const float* x,
                                                              float) {
  const int ib = t >> 1, h = t & 1;
  const uint32_t qh = w[bs + 66 + ib];
  float p = 0.f;
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    const int l = 2 * h + i;
    const size_t q = bs + 2 + 8 * ib + 2 * l;
    const uint32_t i1 = w[q] | ((qh << (8 - 2 * l)) & 256u), i2 = w[q + 1] | ((qh << (7 - 2 * l)) & 256u);
    p = dot8s(iq3s_pair(i1, i2), w[bs + 74 + 4 * ib + l], x + 8 * i, p);
  }
  const uint32_t sc = (w[bs + 106 + (ib >> 1)] >> (4 * (ib & 1))) & 15u;
  return (f16_at(w, bs) * (float)(1 + 2 * sc)) * p;
}

// IQ1 grid entry: 8 values v_j in {-1, 0, 1} stored as v_j + 1 in bits 2 j.. of a u16
__device__ __forceinline__ float iq1_dot(uint32_t e, const float* x, float p) {
#pragma unroll
  for (int j = 0; j < 8; ++j) p = fmaf(x[j], (float)((e >> (2 * j)) & 3u), p);
  return p;
}

// IQ1_S (50 bytes): fp16 d, 32 low index bytes, 8 u16 words qh (3 high index bits per group,
// a 3-bit scale in bits 12-14, the sign of delta in bit 15); value d (2 scale + 1) (grid +- 1/8).
// With the grid stored as v + 1: sum x (v + delta) = sum x (v + 1) + (delta - 1) sum x.
template <> __device__ __forceinline__ float lane_dot<kIQ1_S>(const uint8_t* w, size_t bs, int t, const float* x,
                                                              float xs) {
  const int ib = t >> 1, h = t & 1;
  const uint32_t qh = ld16(w, bs + 34 + 2 * ib);
  float p = 0.f;
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    const int l = 2 * h + i;
    p = iq1_dot(iq::kIQ1S[w[bs + 2 + 4 * ib + l] | (((qh >> (3 * l)) & 7u) << 8)], x + 8 * i, p);
  }
  const float dm1 = (qh & 0x8000u) ? -1.125f : -0.875f;
  return (f16_at(w, bs) * (float)(2 * ((qh >> 12) & 7u) + 1)) * fmaf(dm1, xs, p);
}

// IQ1_M's fp16 block scale: the top nibbles of its four u16 scale words
__device__ __forceinline__ float iq1m_d(const uint8_t* w, size_t bs) {
  const uint32_t s0 = ld16(w, bs + 48), s1 = ld16(w, bs + 50), s2 = ld16(w, bs + 52), s3 = ld16(w, bs + 54);
  const uint32_t u = (s0 >> 12) | ((s1 >> 8) & 0x00F0u) | ((s2 >> 4) & 0x0F00u) | (s3 & 0xF000u);
  return __half2float(__ushort_as_half((unsigned short)u));
}

// IQ1_M (56 bytes): 32 low index bytes, 16 qh bytes (per pair of groups: 3 high bits and a delta
// sign each, bits 0-3 for the first group and 4-7 for the second), 4 u16 scale words (3-bit
// scales, two per sub-block: groups 0-1 and 2-3; the spare top nibbles hold d).
template <> __device__ __forceinline__ float lane_dot<kIQ1_M>(const uint8_t* w, size_t bs, int t, const float* x,
                                                              float) {
  const int ib = t >> 1, h = t & 1;
  const uint32_t qhb = w[bs + 32 + 2 * ib + h];
  const float p0 = iq1_dot(iq::kIQ1S[w[bs + 4 * ib + 2 * h] | ((qhb << 8) & 0x700u)], x, 0.f);
  const float p1 = iq1_dot(iq::kIQ1S[w[bs + 4 * ib + 2 * h + 1] | ((qhb << 4) & 0x700u)], x + 8, 0.f);
  const float s0 = ((x[0] + x[1]) + (x[2] + x[3])) + ((x[4] + x[5]) + (x[6] + x[7]));
  const float s1 = ((x[8] + x[9]) + (x[10] + x[11])) + ((x[12] + x[13]) + (x[14] + x[15]));
  const float p = fmaf((qhb & 0x08u) ? -1.125f : -0.875f, s0, p0) + fmaf((qhb & 0x80u) ? -1.125f : -0.875f, s1, p1);
  const uint32_t sc = ld16(w, bs + 48 + 2 * (ib >> 1)) >> (6 * (ib & 1) + 3 * h);
  return (iq1m_d(w, bs) * (float)(2 * (sc & 7u) + 1)) * p;
}

// ---- ternary, fp4 and 1/2-bit types ----------------------------------------------------------
__device__ __forceinline__ uint32_t pow3(int p) { return p == 0 ? 1u : p == 1 ? 3u : p == 2 ? 9u : p == 3 ? 27u : 81u; }
// the trit a TQ1_0 byte holds at power p: the top of (byte * 3^p mod 256) * 3
__device__ __forceinline__ uint32_t trit(uint32_t b, uint32_t p3) { return (((b * p3) & 0xFFu) * 3u) >> 8; }

// TQ1_0 (54 bytes): qs[48] then qh[4] then fp16 d; five trits per qs byte, four per qh byte.
// Values 0-159: trit p of qs[m] (m < 32) is value 32 p + m; 160-239: trit p of qs[32 + m] is
// value 160 + 16 p + m; 240-255: trit p of qh[j] is value 240 + 4 p + j. Value d (trit - 1).
template <> __device__ __forceinline__ float lane_dot<kTQ1_0>(const uint8_t* w, size_t bs, int t, const float* x,
                                                              float xs) {
  uint32_t c[4];
  load16(w, bs + (t < 10 ? 16 * (t & 1) : 32), c);
  const uint32_t qh = u32_at2(w, bs + 48);
  const uint32_t p3 = pow3(t < 10 ? t >> 1 : t - 10);
  float p = 0.f;
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    const uint32_t b = t == 15 ? (qh >> (8 * (i & 3))) & 0xFFu : (c[i >> 2] >> (8 * (i & 3))) & 0xFFu;
    p = fmaf(x[i], (float)trit(b, t == 15 ? pow3(i >> 2) : p3), p);
  }
  return f16_at(w, bs + 52) * (p - xs);
}

// TQ2_0 (66 bytes): qs[64] then fp16 d; value 128 g + 32 l + m is bits 2 l of qs[32 g + m],
// d (q - 1). Lane t = (g, l, half) takes 16 bytes at 32 g + 16 half.
template <> __device__ __forceinline__ float lane_dot<kTQ2_0>(const uint8_t* w, size_t bs, int t, const float* x,
                                                              float xs) {
  uint32_t c[4];
  load16(w, bs + 32 * (t >> 3) + 16 * (t & 1), c);
  const int l = (t >> 1) & 3;
  float p = 0.f;
#pragma unroll
  for (int i = 0; i < 4; ++i) p = dot4u((c[i] >> (2 * l)) & 0x03030303u, x + 4 * i, p);
  return f16_at(w, bs + 64) * (p - xs);
}

// E2M1 code (doubled: 0 1 2 3 4 6 8 12, negated for codes 8-15) as signed bytes, 4 codes at a time
__device__ __forceinline__ uint32_t fp4_lookup(uint32_t c) {
  const uint32_t sel = c & 0x07070707u;
  const uint32_t a = __builtin_amdgcn_perm(0x0C080604u, 0x03020100u, sel);
  const uint32_t b = __builtin_amdgcn_perm(0xF4F8FAFCu, 0xFDFEFF00u, sel);
  const uint32_t m = ((c >> 3) & 0x01010101u) * 0xFFu;
  return (a & ~m) | (b & m);
}
// four signed bytes against x[0..3]
__device__ __forceinline__ float dot4s(uint32_t v, const float* x, float p) {
#pragma unroll
  for (int j = 0; j < 4; ++j) p = fmaf(x[j], (float)((int)(v << (24 - 8 * j)) >> 24), p);
  return p;
}
// MXFP4's E8M0 exponent e as 2^(e - 128) (the format's scale halved, with the doubled codes)
__device__ __forceinline__ float e8m0_half(uint32_t e) {
  return __uint_as_float(e < 2 ? 0x00200000u << e : (e - 1) << 23);
}
// NVFP4's UE4M3 sub-block scale halved: (8 + m) 2^(e - 11), m 2^-10 when e = 0; 0 and 0x7F give 0
__device__ __forceinline__ float ue4m3_half(uint32_t v) {
  if (v == 0 || v == 0x7Fu) return 0.f;
  const int e = (v >> 3) & 15, m = v & 7;
  return e ? ldexpf((float)(8 + m), e - 11) : ldexpf((float)m, -10);
}

// MXFP4 (17 bytes): E8M0 exponent byte, 16 code bytes (value j < 16: low nibble of byte 1 + j,
// 16 + j: high nibble). Blocks are byte-aligned: the codes are read as bytes.
template <> __device__ __forceinline__ float lane_dot<kMXFP4>(const uint8_t* w, size_t bs, int t, const float* x,
                                                              float) {
  const size_t a = bs + 1 + 8 * (t & 1);
  const uint32_t c0 = w[a] | (w[a + 1] << 8) | (w[a + 2] << 16) | ((uint32_t)w[a + 3] << 24);
  const uint32_t c1 = w[a + 4] | (w[a + 5] << 8) | (w[a + 6] << 16) | ((uint32_t)w[a + 7] << 24);
  const int sh = 4 * (t >> 1);
  const float p = dot4s(fp4_lookup((c1 >> sh) & 0x0F0F0F0Fu), x + 4, dot4s(fp4_lookup((c0 >> sh) & 0x0F0F0F0Fu), x, 0.f));
  return e8m0_half(w[bs]) * p;
}

// NVFP4 (36 bytes): four UE4M3 scale bytes, then per 16-value sub-block s 8 code bytes at
// 4 + 8 s (value 16 s + j: low nibble of byte j < 8, high nibble of byte j - 8).
template <> __device__ __forceinline__ float lane_dot<kNVFP4>(const uint8_t* w, size_t bs, int t, const float* x,
                                                              float) {
  const int s = t >> 1, sh = 4 * (t & 1);
  const uint32_t c0 = ld32(w, bs + 4 + 8 * s), c1 = ld32(w, bs + 8 + 8 * s);
  const float p = dot4s(fp4_lookup((c1 >> sh) & 0x0F0F0F0Fu), x + 4, dot4s(fp4_lookup((c0 >> sh) & 0x0F0F0F0Fu), x, 0.f));
  return ue4m3_half(w[bs + s]) * p;
}

// Q1_0 (18 bytes): fp16 d, one bit per value (bit j % 8 of byte 2 + j / 8): +d when set, else -d.
template <> __device__ __forceinline__ float lane_dot<kQ1_0>(const uint8_t* w, size_t bs, int t, const float* x,
                                                             float xs) {
  const uint32_t b = w[bs + 2 + t];
  float p = 0.f;
#pragma unroll
  for (int j = 0; j < 8; ++j) p = fmaf(x[j], (float)((b >> j) & 1u), p);
  return f16_at(w, bs) * fmaf(2.f, p, -xs);
}

// Q2_0 (18 bytes): fp16 d, two bits per value (bits 2 (j % 4) of byte 2 + j / 4), d (q - 1).
template <> __device__ __forceinline__ float lane_dot<kQ2_0>(const uint8_t* w, size_t bs, int t, const float* x,
                                                             float xs) {
  const uint32_t b = ld16(w, bs + 2 + 2 * t);
  float p = 0.f;
#pragma unroll
  for (int j = 0; j < 8; ++j) p = fmaf(x[j], (float)((b >> (2 * j)) & 3u), p);
  return f16_at(w, bs) * (p - xs);
}

// Grouped expert rows (sparse MoE): grid row m is slot m of a route buffer; its activation row
// is x[sorted_tok[m]] (gather) or x[m], its weight the matrix of the slot's expert (w + e *
// estride, e the last expert whose first slot is <= m), and its result is scaled by the slot's
// routing weight when sorted_w is given. expert_off null: plain rows.
struct Grp {
  const int* expert_off;  // [E + 1] first slot of each expert
  const int* sorted_tok;  // null: row m of x
  const float* sorted_w;  // null: unweighted
  int E;
  size_t estride;
};

// y[m][n] = sum_k x[m][k] * W[n][k] (+ bias[n]); grid (workgroups, M), 256 threads.
template <int T, typename XT, typename OT>
__global__ __launch_bounds__(256) void ggml_gemv_kernel(const XT* __restrict__ x, const uint8_t* __restrict__ w,
                                                        const float* __restrict__ bias, OT* __restrict__ out,
                                                        int K, int N, Grp grp) {
  using B = Blk<T>;
  constexpr int R = B::ROWS, BPP = 64 / B::LPB, VPL = B::VPL;
  extern __shared__ __align__(16) float lds_f[];
  float* xs = lds_f;       // K activations
  float* xg = lds_f + K;   // K / VPL sums of each lane's run
  const int m = blockIdx.y;
  const int lane = threadIdx.x & 63, wave = uniform(threadIdx.x >> 6);
  int xm = m;
  float wsc = 1.f;
  if (grp.expert_off) {  // uniform over the workgroup
    int lo = 0, hi = grp.E;  // expert_off[lo] <= m < expert_off[hi]
    while (hi - lo > 1) {
      const int mid = (lo + hi) >> 1;
      if (grp.expert_off[mid] <= m) lo = mid;
      else hi = mid;
    }
    w += (size_t)uniform(lo) * grp.estride;
    if (grp.sorted_tok) xm = uniform(grp.sorted_tok[m]);
    if (grp.sorted_w) wsc = grp.sorted_w[m];
  }

  // ---- stage the activation row: 8 values per thread, sums of 8 (pairs combined for 16) ----
  for (int i = threadIdx.x; i < K / 8; i += 256) {
    float v[8];
    load8(x + (size_t)xm * K + 8 * i, v);
    float4* d = reinterpret_cast<float4*>(xs + 8 * i);
    d[0] = make_float4(v[0], v[1], v[2], v[3]);
    d[1] = make_float4(v[4], v[5], v[6], v[7]);
    float sum = ((v[0] + v[1]) + (v[2] + v[3])) + ((v[4] + v[5]) + (v[6] + v[7]));
    if constexpr (VPL == 8) {
      xg[i] = sum;
    } else {
      sum += dpp_move<0xB1>(sum);  // i and i ^ 1 are neighbouring lanes (K / 8 is even)
      if ((i & 1) == 0) xg[i >> 1] = sum;
    }
  }
  __syncthreads();

  const int nb = K / B::VALS;
  const size_t row_bytes = (size_t)nb * B::BYTES;
  const int sub = lane / B::LPB, t = lane % B::LPB, kl = lane_k<T>(t);
  const int groups = (N + R - 1) / R;
  const float grp_w = wsc;
  for (int rg = blockIdx.x * 4 + wave; rg < groups; rg += gridDim.x * 4) {
    float acc[R];
#pragma unroll
    for (int r = 0; r < R; ++r) acc[r] = 0.f;
    for (int b0 = 0; b0 < nb; b0 += BPP) {
      const int b = min(b0 + sub, nb - 1);  // lanes past the last block repeat it and add nothing
      const float keep = b0 + sub < nb ? 1.f : 0.f;
      const int k = b * B::VALS + kl;
      float xv[VPL];
#pragma unroll
      for (int i = 0; i < VPL; i += 4) {
        const float4 q = *reinterpret_cast<const float4*>(xs + k + i);
        xv[i] = q.x;
        xv[i + 1] = q.y;
        xv[i + 2] = q.z;
        xv[i + 3] = q.w;
      }
      const float xsum = xg[k / VPL];
#pragma unroll
      for (int r = 0; r < R; ++r) {
        const int n = min(rg * R + r, N - 1);
        acc[r] = fmaf(keep, lane_dot<T>(w, (size_t)n * row_bytes + (size_t)b * B::BYTES, t, xv, xsum), acc[r]);
      }
    }
#pragma unroll
    for (int r = 0; r < R; ++r) acc[r] = wave_sum(acc[r]);
    if (lane < R) {
      float v = acc[0];
#pragma unroll
      for (int r = 1; r < R; ++r)
        if (lane == r) v = acc[r];
      const int n = rg * R + lane;
      if (n < N) {
        if (bias) v += bias[n];
        out[(size_t)m * N + n] = from_f32<OT>(grp_w * v);
      }
    }
  }
}

template <int T, typename XT, typename OT>
static int launch(const void* x, const uint8_t* w, const float* bias, void* out, int M, int K, int N, hipStream_t st,
                  Grp grp = Grp{nullptr, nullptr, nullptr, 0, 0}) {
  auto kern = ggml_gemv_kernel<T, XT, OT>;
  const size_t lds = (size_t)K * 4 + (size_t)(K / Blk<T>::VPL) * 4;
  MIQ_REQUIRE(lds <= 160 * 1024, MIQ_ERR_UNSUPPORTED, "ggml_gemv: K=%d too large to stage", K);
  if (lds > 64 * 1024) {
    const int rc = require_lds("ggml_gemv", lds);
    if (rc) return rc;
  }
  const int groups = (N + Blk<T>::ROWS - 1) / Blk<T>::ROWS;
  int wgs = (groups + 3) / 4;
  if (wgs > 4 * kCUs) wgs = 4 * kCUs;
  hipLaunchKernelGGL(kern, dim3(wgs, M), dim3(256), lds, st, static_cast<const XT*>(x), w, bias,
                     static_cast<OT*>(out), K, N, grp);
  return check_launch("ggml_gemv");
}

template <int T>
static int types(const void* x, int xd, const uint8_t* w, const float* bias, void* out, int od, int M, int K, int N,
                 hipStream_t st) {
  if (xd == MIQ_F16) {
    if (od == MIQ_F16) return launch<T, __half, __half>(x, w, bias, out, M, K, N, st);
    return launch<T, __half, float>(x, w, bias, out, M, K, N, st);
  }
  if (od == MIQ_F16) return launch<T, float, __half>(x, w, bias, out, M, K, N, st);
  return launch<T, float, float>(x, w, bias, out, M, K, N, st);
}

// Value j of a block of the types whose lanes take consecutive values. Each is an exact product
// (a power of two, an fp16 scale times a small odd integer, codebook entries of at most 6 bits,
// codes of at most 2 bits, +-1/8 offsets) so its one rounding is the reference's.
template <int T> __device__ __forceinline__ float value_seq(const uint8_t* w, size_t bs, int j) {
  const int ib = j >> 5, l = (j >> 3) & 3, jj = j & 7;
  if constexpr (T == kQ4_K) {
    const int q = (w[bs + 16 + 32 * (ib >> 1) + (j & 31)] >> (4 * (ib & 1))) & 15;
    int sc, mn;
    scale_min_k4(w, bs + 4, ib, &sc, &mn);
    return (f16_at(w, bs) * (float)sc) * (float)q - f16_at(w, bs + 2) * (float)mn;
  } else if constexpr (T == kIQ2_XXS) {
    const uint32_t a0 = u32_at2(w, bs + 2 + 8 * ib), a1 = u32_at2(w, bs + 6 + 8 * ib);
    const float g = (float)((iq::kIQ2XXS[(a0 >> (8 * l)) & 0xFFu] >> (8 * jj)) & 0xFFu);
    return (f16_at(w, bs) * (0.5f + (float)(a1 >> 28)) * 0.25f) * sgn(g, ksign((a1 >> (7 * l)) & 127u), jj);
  } else if constexpr (T == kIQ2_XS) {
    const uint32_t q = ld16(w, bs + 2 + 2 * (4 * ib + l));
    const float g = (float)((iq::kIQ2XS[q & 511u] >> (8 * jj)) & 0xFFu);
    const uint32_t sc = (w[bs + 66 + ib] >> (4 * (l >> 1))) & 15u;
    return (f16_at(w, bs) * (0.5f + (float)sc) * 0.25f) * sgn(g, ksign(q >> 9), jj);
  } else if constexpr (T == kIQ2_S) {
    const uint32_t idx = w[bs + 2 + 4 * ib + l] | (((uint32_t)w[bs + 66 + ib] << (8 - 2 * l)) & 0x300u);
    const float g = (float)((iq::kIQ2S[idx] >> (8 * jj)) & 0xFFu);
    const uint32_t sc = (w[bs + 74 + ib] >> (4 * (l >> 1))) & 15u;
    return (f16_at(w, bs) * (0.5f + (float)sc) * 0.25f) * sgn(g, w[bs + 34 + 4 * ib + l], jj);
  } else if constexpr (T == kIQ3_XXS) {
    const uint32_t a = u32_at2(w, bs + 66 + 4 * ib);
    const float g = (float)((iq::kIQ3XXS[w[bs + 2 + 8 * ib + 2 * l + (jj >> 2)]] >> (8 * (jj & 3))) & 0xFFu);
    return (f16_at(w, bs) * (0.5f + (float)(a >> 28)) * 0.5f) * sgn(g, ksign((a >> (7 * l)) & 127u), jj);
  } else if constexpr (T == kIQ3_S) {
    const uint32_t qh = w[bs + 66 + ib], e = jj >> 2;
    const uint32_t idx = w[bs + 2 + 8 * ib + 2 * l + e] | ((qh << (8 - 2 * l - e)) & 256u);
    const float g = (float)((iq::kIQ3S[idx] >> (8 * (jj & 3))) & 0xFFu);
    const uint32_t sc = (w[bs + 106 + (ib >> 1)] >> (4 * (ib & 1))) & 15u;
    return (f16_at(w, bs) * (float)(1 + 2 * sc)) * sgn(g, w[bs + 74 + 4 * ib + l], jj);
  } else if constexpr (T == kIQ1_S) {
    const uint32_t qh = ld16(w, bs + 34 + 2 * ib);
    const uint32_t e = iq::kIQ1S[w[bs + 2 + 4 * ib + l] | (((qh >> (3 * l)) & 7u) << 8)];
    const float v = (float)((int)((e >> (2 * jj)) & 3u) - 1) + ((qh & 0x8000u) ? -0.125f : 0.125f);
    return (f16_at(w, bs) * (float)(2 * ((qh >> 12) & 7u) + 1)) * v;
  } else if constexpr (T == kIQ1_M) {
    const uint32_t qhb = w[bs + 32 + 2 * ib + (l >> 1)];
    const uint32_t idx = w[bs + 4 * ib + l] | ((qhb << ((l & 1) ? 4 : 8)) & 0x700u);
    const uint32_t e = iq::kIQ1S[idx];
    const uint32_t neg = (l & 1) ? (qhb & 0x80u) : (qhb & 0x08u);
    const float v = (float)((int)((e >> (2 * jj)) & 3u) - 1) + (neg ? -0.125f : 0.125f);
    const uint32_t sc = ld16(w, bs + 48 + 2 * (ib >> 1)) >> (6 * (ib & 1) + 3 * (l >> 1));
    return (iq1m_d(w, bs) * (float)(2 * (sc & 7u) + 1)) * v;
  } else if constexpr (T == kTQ1_0) {
    uint32_t b, p;
    if (j < 160) { b = w[bs + (j & 31)]; p = (uint32_t)j >> 5; }
    else if (j < 240) { b = w[bs + 32 + ((j - 160) & 15)]; p = (uint32_t)(j - 160) >> 4; }
    else { b = w[bs + 48 + ((j - 240) & 3)]; p = (uint32_t)(j - 240) >> 2; }
    return (float)((int)trit(b, pow3((int)p)) - 1) * f16_at(w, bs + 52);
  } else if constexpr (T == kTQ2_0) {
    const int g = j >> 7, r = j & 127;
    return (float)((int)((w[bs + 32 * g + (r & 31)] >> (2 * (r >> 5))) & 3u) - 1) * f16_at(w, bs + 64);
  } else if constexpr (T == kMXFP4) {
    const uint32_t q = (w[bs + 1 + (j & 15)] >> (4 * (j >> 4))) & 15u;
    return (float)((int)(fp4_lookup(q) << 24) >> 24) * e8m0_half(w[bs]);
  } else if constexpr (T == kNVFP4) {
    const int sb = j >> 4, r = j & 15;
    const uint32_t q = (w[bs + 4 + 8 * sb + (r & 7)] >> (4 * (r >> 3))) & 15u;
    return (float)((int)(fp4_lookup(q) << 24) >> 24) * ue4m3_half(w[bs + sb]);
  } else if constexpr (T == kQ1_0) {
    const float d = f16_at(w, bs);
    return ((w[bs + 2 + (j >> 3)] >> (j & 7)) & 1u) ? d : -d;
  } else {  // Q2_0
    return (float)((int)((w[bs + 2 + (j >> 2)] >> (2 * (j & 3))) & 3u) - 1) * f16_at(w, bs);
  }
}

// Value j of the block at bs. Every value is an exact product (fp16 scale, small integer
// sub-scale and code fit float32's 24 bits) or such a product plus/minus another exact one, so
// its one rounding matches the reference's numpy whatever the order of the factors.
__device__ __constant__ float kIQ4[16] = {-127.f, -104.f, -83.f, -65.f, -49.f, -35.f, -22.f, -10.f,
                                         1.f,    13.f,   25.f,  38.f,  53.f,  69.f,  89.f,  113.f};
template <int T> __device__ __forceinline__ float value_at(const uint8_t* w, size_t bs, int j) {
  if constexpr (SeqLanes<T>::value) {
    return value_seq<T>(w, bs, j);
  } else if constexpr (T == kQ8_0) {
    return f16_at(w, bs) * (float)(int8_t)w[bs + 2 + j];
  } else if constexpr (T == kQ6_K) {
    const int h = j >> 7, r = j & 127, q = r >> 5, l = r & 31;
    const uint32_t lo = w[bs + 64 * h + l + 32 * (q & 1)];
    const uint32_t nib = (q >> 1) ? (lo >> 4) : (lo & 15u);
    const uint32_t c = nib | (((uint32_t)(w[bs + 128 + 32 * h + l] >> (2 * q)) & 3u) << 4);
    const float sc = (float)(int8_t)w[bs + 192 + 8 * h + (l >> 4) + 2 * q];
    return (f16_at(w, bs + 208) * sc) * (float)((int)c - 32);
  } else if constexpr (Blk<T>::VALS == 32) {  // value j: nibble j >> 4 of code byte j & 15
    constexpr int QS = T == kQ4_0 || T == kIQ4_NL ? 2 : T == kQ4_1 ? 4 : T == kQ5_0 ? 6 : 8;
    int q = (w[bs + QS + (j & 15)] >> (4 * (j >> 4))) & 15;
    if constexpr (T == kQ5_0 || T == kQ5_1) q |= (int)((u32_at2(w, bs + QS - 4) >> j) & 1u) << 4;
    const float d = f16_at(w, bs);
    if constexpr (T == kQ4_0) return d * (float)(q - 8);
    else if constexpr (T == kQ5_0) return d * (float)(q - 16);
    else if constexpr (T == kIQ4_NL) return d * kIQ4[q];
    else return d * (float)q + f16_at(w, bs + 2);  // Q4_1, Q5_1: d * q + m
  } else if constexpr (T == kIQ4_XS) {
    const int ib = j >> 5, q = (w[bs + 8 + 16 * ib + (j & 15)] >> (4 * ((j >> 4) & 1))) & 15;
    const int ls = ((w[bs + 4 + ib / 2] >> (4 * (ib & 1))) & 15) | (((int)(ld16(w, bs + 2) >> (2 * ib)) & 3) << 4);
    return (f16_at(w, bs) * (float)(ls - 32)) * kIQ4[q];
  } else if constexpr (T == kQ5_K) {
    const int sb = j >> 5, l = j & 31;
    const int q = ((w[bs + 48 + 32 * (sb >> 1) + l] >> (4 * (sb & 1))) & 15) + 16 * ((w[bs + 16 + l] >> sb) & 1);
    int sc, mn;
    scale_min_k4(w, bs + 4, sb, &sc, &mn);
    return (f16_at(w, bs) * (float)sc) * (float)q - f16_at(w, bs + 2) * (float)mn;
  } else {  // Q2_K, Q3_K: value 128 h + 32 jj + 16 u + l
    const int h = j >> 7, jj = (j >> 5) & 3, u = (j >> 4) & 1, l = j & 15, is = 8 * h + 2 * jj + u;
    if constexpr (T == kQ2_K) {
      const int q = (w[bs + 16 + 32 * h + 16 * u + l] >> (2 * jj)) & 3;
      const int sc = w[bs + is];
      return (f16_at(w, bs + 80) * (float)(sc & 15)) * (float)q - f16_at(w, bs + 82) * (float)(sc >> 4);
    } else {
      const int q = ((w[bs + 32 + 32 * h + 16 * u + l] >> (2 * jj)) & 3) - (((w[bs + 16 * u + l] >> (4 * h + jj)) & 1) ? 0 : 4);
      const int sc = (((int)w[bs + 96 + (is & 7)] >> (4 * (is >> 3))) & 15) |
                     ((((int)w[bs + 104 + (is & 3)] >> (2 * (is >> 2))) & 3) << 4);
      return (f16_at(w, bs + 108) * (float)(sc - 32)) * (float)q;
    }
  }
}

// Full fp32 dequant of n_blocks blocks, one thread per weight.
template <int T>
__global__ __launch_bounds__(256) void ggml_dequant_kernel(const uint8_t* __restrict__ w, float* __restrict__ out,
                                                           int64_t nvals) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= nvals) return;
  const int64_t blk = i / Blk<T>::VALS;
  out[i] = value_at<T>(w, (size_t)blk * Blk<T>::BYTES, (int)(i - blk * Blk<T>::VALS));
}

// Calls f(std::integral_constant<int, T>) for the native type id t; false if t is not one.
template <typename F> static bool with_type(int t, F&& f) {
  switch (t) {
#define MIQ_GG_CASE(X) \
  case X:              \
    f(std::integral_constant<int, X>{}); \
    return true;
    MIQ_GG_CASE(kQ8_0) MIQ_GG_CASE(kQ6_K) MIQ_GG_CASE(kQ4_0) MIQ_GG_CASE(kQ4_1) MIQ_GG_CASE(kQ5_0)
    MIQ_GG_CASE(kQ5_1) MIQ_GG_CASE(kIQ4_NL) MIQ_GG_CASE(kIQ4_XS) MIQ_GG_CASE(kQ5_K) MIQ_GG_CASE(kQ2_K)
    MIQ_GG_CASE(kQ3_K) MIQ_GG_CASE(kIQ2_XXS) MIQ_GG_CASE(kIQ2_XS) MIQ_GG_CASE(kIQ2_S) MIQ_GG_CASE(kIQ3_XXS)
    MIQ_GG_CASE(kIQ3_S) MIQ_GG_CASE(kIQ1_S) MIQ_GG_CASE(kIQ1_M) MIQ_GG_CASE(kTQ1_0) MIQ_GG_CASE(kTQ2_0)
    MIQ_GG_CASE(kMXFP4) MIQ_GG_CASE(kNVFP4) MIQ_GG_CASE(kQ1_0) MIQ_GG_CASE(kQ2_0) MIQ_GG_CASE(kQ4_K)
#undef MIQ_GG_CASE
    default: return false;
  }
}

// ---- unquantized 2-D weights (GGUF F32 / F16 / BF16 matrices, multiplied as stored) ----------
template <int T> struct Dense;
template <> struct Dense<kF32> { static constexpr int ESZ = 4; };
template <> struct Dense<kF16> { static constexpr int ESZ = 2; };
template <> struct Dense<kBF16> { static constexpr int ESZ = 2; };
// element i of a row of T values
template <int T> __device__ __forceinline__ float dense_at(const uint8_t* w, size_t i) {
  if constexpr (T == kF32) return __uint_as_float(ld32(w, 4 * i));
  else if constexpr (T == kF16) return f16_at(w, 2 * i);
  else return __uint_as_float(ld16(w, 2 * i) << 16);
}
// the 8 (2-byte types) or 4 (F32) values of a 16-byte word
template <int T> __device__ __forceinline__ void dense16(uint4 q, float* v) {
  const uint32_t u[4] = {q.x, q.y, q.z, q.w};
  if constexpr (T == kF32) {
#pragma unroll
    for (int i = 0; i < 4; ++i) v[i] = __uint_as_float(u[i]);
  } else {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      if constexpr (T == kF16) {
        v[2 * i] = __half2float(__ushort_as_half((unsigned short)(u[i] & 0xFFFFu)));
        v[2 * i + 1] = __half2float(__ushort_as_half((unsigned short)(u[i] >> 16)));
      } else {
        v[2 * i] = __uint_as_float(u[i] << 16);
        v[2 * i + 1] = __uint_as_float(u[i] & 0xFFFF0000u);
      }
    }
  }
}

// y[m][n] = sum_k x[m][k] * W[n][k] (+ bias[n]) with W's N rows of K values as stored; grid
// (workgroups, M), 256 threads, each wave two rows at a time. When a row is a whole number of
// 16-byte words (VEC) lanes take 16-byte words, else single values.
template <int T, bool VEC, typename XT, typename OT>
__global__ __launch_bounds__(256) void dense_gemv_kernel(const XT* __restrict__ x, const uint8_t* __restrict__ w,
                                                         const float* __restrict__ bias, OT* __restrict__ out, int K,
                                                         int N) {
  constexpr int ESZ = Dense<T>::ESZ, PW = 16 / ESZ;  // values per 16-byte word
  extern __shared__ __align__(16) float lds_f[];
  const int m = blockIdx.y;
  const int lane = threadIdx.x & 63, wave = uniform(threadIdx.x >> 6);
  for (int i = threadIdx.x; i < K; i += 256) lds_f[i] = to_f32(x[(size_t)m * K + i]);
  __syncthreads();
  const size_t row_bytes = (size_t)K * ESZ;
  const int pairs = (N + 1) / 2;
  for (int pr = blockIdx.x * 4 + wave; pr < pairs; pr += gridDim.x * 4) {
    const int n0 = 2 * pr, n1 = min(2 * pr + 1, N - 1);
    float a0 = 0.f, a1 = 0.f;
    if constexpr (VEC) {
      const int words = K / PW;
      for (int c = lane; c < words; c += 64) {
        float v0[PW], v1[PW];
        dense16<T>(*reinterpret_cast<const uint4*>(w + (size_t)n0 * row_bytes + 16 * (size_t)c), v0);
        dense16<T>(*reinterpret_cast<const uint4*>(w + (size_t)n1 * row_bytes + 16 * (size_t)c), v1);
#pragma unroll
        for (int i = 0; i < PW; ++i) {
          const float xv = lds_f[PW * c + i];
          a0 = fmaf(xv, v0[i], a0);
          a1 = fmaf(xv, v1[i], a1);
        }
      }
    } else {
      for (int k = lane; k < K; k += 64) {
        const float xv = lds_f[k];
        a0 = fmaf(xv, dense_at<T>(w + (size_t)n0 * row_bytes, k), a0);
        a1 = fmaf(xv, dense_at<T>(w + (size_t)n1 * row_bytes, k), a1);
      }
    }
    a0 = wave_sum(a0);
    a1 = wave_sum(a1);
    if (lane < 2) {
      const int n = lane ? 2 * pr + 1 : n0;
      float v = lane ? a1 : a0;
      if (n < N) {
        if (bias) v += bias[n];
        out[(size_t)m * N + n] = from_f32<OT>(v);
      }
    }
  }
}

template <int T, typename XT, typename OT>
static int dense_launch(const void* x, const uint8_t* w, const float* bias, void* out, int M, int K, int N,
                        hipStream_t st) {
  const size_t lds = (size_t)K * 4;
  MIQ_REQUIRE(lds <= 160 * 1024, MIQ_ERR_UNSUPPORTED, "ggml_gemv: K=%d too large to stage", K);
  const bool vec = ((size_t)K * Dense<T>::ESZ) % 16 == 0;
  auto kern = vec ? dense_gemv_kernel<T, true, XT, OT> : dense_gemv_kernel<T, false, XT, OT>;
  if (lds > 64 * 1024) {
    const int rc = require_lds("ggml_gemv", lds);
    if (rc) return rc;
  }
  int wgs = ((N + 1) / 2 + 3) / 4;
  if (wgs > 4 * kCUs) wgs = 4 * kCUs;
  hipLaunchKernelGGL(kern, dim3(wgs, M), dim3(256), lds, st, static_cast<const XT*>(x), w, bias,
                     static_cast<OT*>(out), K, N);
  return check_launch("ggml_gemv");
}

template <int T>
static int dense_types(const void* x, int xd, const uint8_t* w, const float* bias, void* out, int od, int M, int K,
                       int N, hipStream_t st) {
  if (xd == MIQ_F16) {
    if (od == MIQ_F16) return dense_launch<T, __half, __half>(x, w, bias, out, M, K, N, st);
    return dense_launch<T, __half, float>(x, w, bias, out, M, K, N, st);
  }
  if (od == MIQ_F16) return dense_launch<T, float, __half>(x, w, bias, out, M, K, N, st);
  return dense_launch<T, float, float>(x, w, bias, out, M, K, N, st);
}

// fp32 copy of n stored values (the widening is exact)
template <int T>
__global__ __launch_bounds__(256) void dense_dequant_kernel(const uint8_t* __restrict__ w, float* __restrict__ out,
                                                            int64_t n) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i < n) out[i] = dense_at<T>(w, (size_t)i);
}

template <typename F> static bool with_dense(int t, F&& f) {
  switch (t) {
    case kF32: f(std::integral_constant<int, kF32>{}); return true;
    case kF16: f(std::integral_constant<int, kF16>{}); return true;
    case kBF16: f(std::integral_constant<int, kBF16>{}); return true;
    default: return false;
  }
}

}  // namespace gg
}  // namespace miq

using namespace miq;

extern "C" int miq_ggml_dequant_f32(const uint8_t* blocks, int ggml_type, float* out, int64_t n_blocks,
                                    void* stream) {
  if (ggml_type == 12) return miq_q4k_dequant_f32(blocks, out, n_blocks, stream);
  MIQ_REQUIRE(n_blocks >= 0, MIQ_ERR_INVALID, "ggml_dequant: n_blocks=%lld", (long long)n_blocks);
  if (gg::with_dense(ggml_type, [](auto) {})) {  // one value per block
    if (n_blocks == 0) return MIQ_OK;
    MIQ_REQUIRE(blocks && out, MIQ_ERR_INVALID, "ggml_dequant: null pointer");
    MIQ_REQUIRE(aligned(blocks, ggml_type == gg::kF32 ? 4 : 2), MIQ_ERR_ALIGN, "ggml_dequant: misaligned values");
    hipStream_t st = static_cast<hipStream_t>(stream);
    gg::with_dense(ggml_type, [&](auto tag) {
      hipLaunchKernelGGL(gg::dense_dequant_kernel<decltype(tag)::value>, dim3((unsigned)((n_blocks + 255) / 256)),
                         dim3(256), 0, st, blocks, out, n_blocks);
    });
    return check_launch("ggml_dequant");
  }
  int vals = 0;
  const bool known = gg::with_type(ggml_type, [&](auto tag) { vals = gg::Blk<decltype(tag)::value>::VALS; });
  MIQ_REQUIRE(known, MIQ_ERR_UNSUPPORTED, "ggml_dequant: ggml type %d has no native decoder", ggml_type);
  if (n_blocks == 0) return MIQ_OK;
  MIQ_REQUIRE(blocks && out, MIQ_ERR_INVALID, "ggml_dequant: null pointer");
  MIQ_REQUIRE(aligned(blocks, 2), MIQ_ERR_ALIGN, "ggml_dequant: blocks must be 2-byte aligned");
  hipStream_t st = static_cast<hipStream_t>(stream);
  const int64_t nv = n_blocks * vals;
  gg::with_type(ggml_type, [&](auto tag) {
    hipLaunchKernelGGL(gg::ggml_dequant_kernel<decltype(tag)::value>, dim3((unsigned)((nv + 255) / 256)), dim3(256),
                       0, st, blocks, out, nv);
  });
  return check_launch("ggml_dequant");
}

extern "C" int miq_ggml_gemv(const void* x, int x_dtype, const uint8_t* w, int ggml_type, const float* bias,
                             void* out, int out_dtype, int M, int K, int N, void* stream) {
  int vals = 0;
  const bool dense = gg::with_dense(ggml_type, [](auto) {});
  const bool known = dense || gg::with_type(ggml_type, [&](auto tag) { vals = gg::Blk<decltype(tag)::value>::VALS; });
  MIQ_REQUIRE(known, MIQ_ERR_UNSUPPORTED, "ggml_gemv: ggml type %d has no kernel here (Q4_K: miq_q4k_gemv)",
              ggml_type);
  if (dense) vals = 1;
  MIQ_REQUIRE(M >= 0 && K > 0 && N > 0 && M <= 65535, MIQ_ERR_INVALID, "ggml_gemv: M=%d K=%d N=%d", M, K, N);
  MIQ_REQUIRE(K % vals == 0, MIQ_ERR_INVALID, "ggml_gemv: K=%d is not a multiple of %d", K, vals);
  if (M == 0) return MIQ_OK;
  MIQ_REQUIRE(x && w && out, MIQ_ERR_INVALID, "ggml_gemv: null pointer");
  MIQ_REQUIRE(aligned(w, 16) && aligned(x, 16), MIQ_ERR_ALIGN, "ggml_gemv: x and weight must be 16-byte aligned");
  MIQ_REQUIRE(x_dtype == MIQ_F16 || x_dtype == MIQ_F32, MIQ_ERR_UNSUPPORTED, "ggml_gemv: x dtype");
  MIQ_REQUIRE(out_dtype == MIQ_F16 || out_dtype == MIQ_F32, MIQ_ERR_UNSUPPORTED, "ggml_gemv: out dtype");
  hipStream_t st = static_cast<hipStream_t>(stream);
  int rc = MIQ_OK;
  if (dense) {
    gg::with_dense(ggml_type, [&](auto tag) {
      rc = gg::dense_types<decltype(tag)::value>(x, x_dtype, w, bias, out, out_dtype, M, K, N, st);
    });
    return rc;
  }
  gg::with_type(ggml_type, [&](auto tag) {
    rc = gg::types<decltype(tag)::value>(x, x_dtype, w, bias, out, out_dtype, M, K, N, st);
  });
  return rc;
}

extern "C" int miq_moe_ggml_gemv(const void* x, int x_dtype, const void* route, int T, int E, int k, int gather,
                                 int weighted, const uint8_t* w, int ggml_type, size_t expert_stride, float* out,
                                 int K, int N, void* stream) {
  int vals = 0, bytes = 0;
  const bool known = gg::with_type(ggml_type, [&](auto tag) {
    vals = gg::Blk<decltype(tag)::value>::VALS;
    bytes = gg::Blk<decltype(tag)::value>::BYTES;
  });
  MIQ_REQUIRE(known, MIQ_ERR_UNSUPPORTED, "moe_ggml_gemv: ggml type %d has no block kernel", ggml_type);
  MIQ_REQUIRE(T >= 0 && E > 0 && E <= 1024 && k > 0 && k <= E && (size_t)T * k <= (size_t)kMoeMaxTK && K > 0 && N > 0,
              MIQ_ERR_INVALID, "moe_ggml_gemv: T=%d E=%d k=%d K=%d N=%d", T, E, k, K, N);
  MIQ_REQUIRE(K % vals == 0, MIQ_ERR_INVALID, "moe_ggml_gemv: K=%d is not a multiple of %d", K, vals);
  MIQ_REQUIRE(expert_stride >= (size_t)N * (K / vals) * bytes, MIQ_ERR_INVALID,
              "moe_ggml_gemv: expert stride %zu below one expert's %zu bytes", expert_stride,
              (size_t)N * (K / vals) * bytes);
  if (T == 0) return MIQ_OK;
  MIQ_REQUIRE(x && route && w && out, MIQ_ERR_INVALID, "moe_ggml_gemv: null pointer");
  // an expert is a whole number of blocks, so its rows keep the block alignment the lane loads
  // assume (2 bytes; 4 for NVFP4; MXFP4 reads bytes)
  MIQ_REQUIRE(aligned(w, 16) && aligned(x, 16) && aligned(route, 16) &&
                  (ggml_type == gg::kMXFP4 || expert_stride % 4 == 0),
              MIQ_ERR_ALIGN, "moe_ggml_gemv: x, weights, route 16-byte aligned, expert stride a multiple of 4");
  MIQ_REQUIRE(x_dtype == MIQ_F16 || x_dtype == MIQ_F32, MIQ_ERR_UNSUPPORTED, "moe_ggml_gemv: x dtype");
  const RouteLayout L = route_layout(T, E, k);
  const int* r = static_cast<const int*>(route);
  gg::Grp grp{r + L.expert_off, gather ? r + L.sorted_tok : nullptr,
              weighted ? reinterpret_cast<const float*>(r + L.sorted_w) : nullptr, E, expert_stride};
  hipStream_t st = static_cast<hipStream_t>(stream);
  int rc = MIQ_OK;
  gg::with_type(ggml_type, [&](auto tag) {
    constexpr int TT = decltype(tag)::value;
    rc = x_dtype == MIQ_F16 ? gg::launch<TT, __half, float>(x, w, nullptr, out, T * k, K, N, st, grp)
                            : gg::launch<TT, float, float>(x, w, nullptr, out, T * k, K, N, st, grp);
  });
  return rc;
}
