// GGUF Q8_0 and Q6_K: decode GEMV over the native blocks (gfx950), the types a Q4_K_M file
// mixes in beside Q4_K.
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

namespace miq {
namespace gg {

constexpr int kQ8_0 = 8, kQ6_K = 14;  // ggml type ids

template <int T> struct Blk;
template <> struct Blk<kQ8_0> {
  static constexpr int VALS = 32, BYTES = 34, LPB = 4, VPL = 8;
};
template <> struct Blk<kQ6_K> {
  static constexpr int VALS = 256, BYTES = 210, LPB = 16, VPL = 16;
};

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

// Position of lane t's first weight within its block.
template <int T> __device__ __forceinline__ int lane_k(int t) {
  if constexpr (T == kQ8_0) return 8 * t;
  else return 128 * (t >> 3) + 32 * ((t >> 1) & 3) + 16 * (t & 1);
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

// y[m][n] = sum_k x[m][k] * W[n][k] (+ bias[n]); grid (workgroups, M), 256 threads.
template <int T, typename XT, typename OT>
__global__ __launch_bounds__(256) void ggml_gemv_kernel(const XT* __restrict__ x, const uint8_t* __restrict__ w,
                                                        const float* __restrict__ bias, OT* __restrict__ out,
                                                        int K, int N) {
  using B = Blk<T>;
  constexpr int R = 4, BPP = 64 / B::LPB, VPL = B::VPL;
  extern __shared__ __align__(16) float lds_f[];
  float* xs = lds_f;       // K activations
  float* xg = lds_f + K;   // K / VPL sums of each lane's run
  const int m = blockIdx.y;
  const int lane = threadIdx.x & 63, wave = uniform(threadIdx.x >> 6);

  // ---- stage the activation row: 8 values per thread, sums of 8 (pairs combined for 16) ----
  for (int i = threadIdx.x; i < K / 8; i += 256) {
    float v[8];
    load8(x + (size_t)m * K + 8 * i, v);
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
  for (int grp = blockIdx.x * 4 + wave; grp < groups; grp += gridDim.x * 4) {
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
        const int n = min(grp * R + r, N - 1);
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
      const int n = grp * R + lane;
      if (n < N) {
        if (bias) v += bias[n];
        out[(size_t)m * N + n] = from_f32<OT>(v);
      }
    }
  }
}

template <int T, typename XT, typename OT>
static int launch(const void* x, const uint8_t* w, const float* bias, void* out, int M, int K, int N, hipStream_t st) {
  auto kern = ggml_gemv_kernel<T, XT, OT>;
  const size_t lds = (size_t)K * 4 + (size_t)(K / Blk<T>::VPL) * 4;
  MIQ_REQUIRE(lds <= 160 * 1024, MIQ_ERR_UNSUPPORTED, "ggml_gemv: K=%d too large to stage", K);
  if (lds > 64 * 1024) {
    const int rc = require_lds("ggml_gemv", lds);
    if (rc) return rc;
  }
  const int groups = (N + 3) / 4;
  int wgs = (groups + 3) / 4;
  if (wgs > 4 * kCUs) wgs = 4 * kCUs;
  hipLaunchKernelGGL(kern, dim3(wgs, M), dim3(256), lds, st, static_cast<const XT*>(x), w, bias,
                     static_cast<OT*>(out), K, N);
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

// Full fp32 dequant of n_blocks blocks, one thread per weight. Every product is exact in fp32
// (fp16 d x int8 code; fp16 d x int8 scale x 6-bit code), so the order of the factors does
// not change a bit.
template <int T>
__global__ __launch_bounds__(256) void ggml_dequant_kernel(const uint8_t* __restrict__ w, float* __restrict__ out,
                                                           int64_t nvals) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= nvals) return;
  const int64_t blk = i / Blk<T>::VALS;
  const int j = (int)(i - blk * Blk<T>::VALS);
  const size_t bs = (size_t)blk * Blk<T>::BYTES;
  if constexpr (T == kQ8_0) {
    out[i] = f16_at(w, bs) * (float)(int8_t)w[bs + 2 + j];
  } else {
    const int h = j >> 7, r = j & 127, q = r >> 5, l = r & 31;
    const uint32_t lo = w[bs + 64 * h + l + 32 * (q & 1)];
    const uint32_t nib = (q >> 1) ? (lo >> 4) : (lo & 15u);
    const uint32_t c = nib | (((uint32_t)(w[bs + 128 + 32 * h + l] >> (2 * q)) & 3u) << 4);
    const float sc = (float)(int8_t)w[bs + 192 + 8 * h + (l >> 4) + 2 * q];
    out[i] = (f16_at(w, bs + 208) * sc) * (float)((int)c - 32);
  }
}

}  // namespace gg
}  // namespace miq

using namespace miq;

extern "C" int miq_ggml_dequant_f32(const uint8_t* blocks, int ggml_type, float* out, int64_t n_blocks,
                                    void* stream) {
  if (ggml_type == 12) return miq_q4k_dequant_f32(blocks, out, n_blocks, stream);
  MIQ_REQUIRE(ggml_type == gg::kQ8_0 || ggml_type == gg::kQ6_K, MIQ_ERR_UNSUPPORTED,
              "ggml_dequant: ggml type %d (Q4_K = 12, Q8_0 = 8 and Q6_K = 14 are decoded here)", ggml_type);
  MIQ_REQUIRE(n_blocks >= 0, MIQ_ERR_INVALID, "ggml_dequant: n_blocks=%lld", (long long)n_blocks);
  if (n_blocks == 0) return MIQ_OK;
  MIQ_REQUIRE(blocks && out, MIQ_ERR_INVALID, "ggml_dequant: null pointer");
  MIQ_REQUIRE(aligned(blocks, 2), MIQ_ERR_ALIGN, "ggml_dequant: blocks must be 2-byte aligned");
  hipStream_t st = static_cast<hipStream_t>(stream);
  const int64_t vals = n_blocks * (ggml_type == gg::kQ8_0 ? 32 : 256);
  const dim3 grid((unsigned)((vals + 255) / 256));
  if (ggml_type == gg::kQ8_0) hipLaunchKernelGGL(gg::ggml_dequant_kernel<gg::kQ8_0>, grid, dim3(256), 0, st, blocks, out, vals);
  else hipLaunchKernelGGL(gg::ggml_dequant_kernel<gg::kQ6_K>, grid, dim3(256), 0, st, blocks, out, vals);
  return check_launch("ggml_dequant");
}

extern "C" int miq_ggml_gemv(const void* x, int x_dtype, const uint8_t* w, int ggml_type, const float* bias,
                             void* out, int out_dtype, int M, int K, int N, void* stream) {
  MIQ_REQUIRE(ggml_type == gg::kQ8_0 || ggml_type == gg::kQ6_K, MIQ_ERR_UNSUPPORTED,
              "ggml_gemv: ggml type %d (Q8_0 = 8 and Q6_K = 14 are decoded here, Q4_K by miq_q4k_gemv)",
              ggml_type);
  const int vals = ggml_type == gg::kQ8_0 ? 32 : 256;
  MIQ_REQUIRE(M >= 0 && K > 0 && N > 0 && M <= 65535, MIQ_ERR_INVALID, "ggml_gemv: M=%d K=%d N=%d", M, K, N);
  MIQ_REQUIRE(K % vals == 0, MIQ_ERR_INVALID, "ggml_gemv: K=%d is not a multiple of %d", K, vals);
  if (M == 0) return MIQ_OK;
  MIQ_REQUIRE(x && w && out, MIQ_ERR_INVALID, "ggml_gemv: null pointer");
  MIQ_REQUIRE(aligned(w, 16) && aligned(x, 16), MIQ_ERR_ALIGN, "ggml_gemv: x and weight must be 16-byte aligned");
  MIQ_REQUIRE(x_dtype == MIQ_F16 || x_dtype == MIQ_F32, MIQ_ERR_UNSUPPORTED, "ggml_gemv: x dtype");
  MIQ_REQUIRE(out_dtype == MIQ_F16 || out_dtype == MIQ_F32, MIQ_ERR_UNSUPPORTED, "ggml_gemv: out dtype");
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (ggml_type == gg::kQ8_0) return gg::types<gg::kQ8_0>(x, x_dtype, w, bias, out, out_dtype, M, K, N, st);
  return gg::types<gg::kQ6_K>(x, x_dtype, w, bias, out, out_dtype, M, K, N, st);
}
