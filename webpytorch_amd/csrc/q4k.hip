// GGUF Q4_K: fp32 dequant and decode GEMV over the native 144-byte super-blocks (gfx950).
//
// Super-block (256 weights, 144 bytes): fp16 d at 0, fp16 dmin at 2, 12 bytes of packed
// 6-bit sub-block scales/mins at 4, 128 bytes of 4-bit codes at 16. Sub-block j (32 weights)
// dequantizes as (d * sc[j]) * code - (dmin * m[j]); byte i of the 32-byte code group
// q = j / 2 holds weight i of sub-block 2q (low nibble) and of 2q+1 (high nibble).
// A weight matrix is N rows of K/256 consecutive super-blocks, exactly as the file holds it.
//
// GEMV mapping: four lanes share a super-block, lane (b, q) owning its 32-byte code group
// (64 weights, two sub-blocks), so a wave covers 16 super-blocks (4096 activations) of a row
// with 16-byte loads; the lane keeps its 64 activations in registers and walks R rows.
#include "miq_common.h"

namespace miq {

struct Q4kScales {
  float d1, m1, d2, m2;  // d*sc and dmin*m for sub-blocks 2q and 2q+1
};

// Decode the two sub-block scale/min pairs of code group q from the 16-byte header.
__device__ __forceinline__ Q4kScales q4k_scales(uint4 h, int q) {
  const float d = __half2float(__ushort_as_half((unsigned short)(h.x & 0xFFFF)));
  const float dmin = __half2float(__ushort_as_half((unsigned short)(h.x >> 16)));
  // header bytes 4..15 are the 12 packed scale bytes s[0..11] = words y (s0-3), z (s4-7), w (s8-11)
  uint32_t sc[2], mn[2];
#pragma unroll
  for (int t = 0; t < 2; ++t) {
    const int j = 2 * q + t;
    const int sh = (j & 3) * 8;
    const uint32_t a = (h.y >> sh) & 0xFF;  // s[j & 3]
    const uint32_t b = (h.z >> sh) & 0xFF;  // s[(j & 3) + 4]
    const uint32_t c = (h.w >> sh) & 0xFF;  // s[(j & 3) + 8]
    const uint32_t lo_sc = a & 63, lo_m = b & 63;
    const uint32_t hi_sc = (c & 15) | ((a >> 6) << 4);
    const uint32_t hi_m = (c >> 4) | ((b >> 6) << 4);
    sc[t] = j < 4 ? lo_sc : hi_sc;
    mn[t] = j < 4 ? lo_m : hi_m;
  }
  Q4kScales r;
  r.d1 = d * (float)sc[0];
  r.m1 = dmin * (float)mn[0];
  r.d2 = d * (float)sc[1];
  r.m2 = dmin * (float)mn[1];
  return r;
}

// fp32 dequant: one thread per (super-block, code group) writes 64 values.
__global__ __launch_bounds__(256) void q4k_dequant_kernel(const uint8_t* __restrict__ blocks,
                                                          float* __restrict__ out, int64_t n_blocks) {
  const int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int64_t b = t >> 2;
  const int q = (int)(t & 3);
  if (b >= n_blocks) return;
  const uint8_t* blk = blocks + b * 144;
  const uint4 h = *reinterpret_cast<const uint4*>(blk);
  const Q4kScales s = q4k_scales(h, q);
  const uint4 c0 = *reinterpret_cast<const uint4*>(blk + 16 + 32 * q);
  const uint4 c1 = *reinterpret_cast<const uint4*>(blk + 32 + 32 * q);
  const uint32_t cw[8] = {c0.x, c0.y, c0.z, c0.w, c1.x, c1.y, c1.z, c1.w};
  float* o = out + b * 256 + 64 * q;
#pragma unroll
  for (int i = 0; i < 32; ++i) {
    const uint32_t byte = (cw[i >> 2] >> ((i & 3) * 8)) & 0xFF;
    o[i] = fmaf(s.d1, (float)(byte & 15), -s.m1);
    o[32 + i] = fmaf(s.d2, (float)(byte >> 4), -s.m2);
  }
}

// y[m][n] = sum_k x[m][k] * W[n][k]  (+ bias[n])
template <int R, int MR, typename XT, typename OT>
__global__ __launch_bounds__(256) void q4k_gemv_kernel(const XT* __restrict__ x, const uint8_t* __restrict__ w,
                                                       const float* __restrict__ bias, OT* __restrict__ out,
                                                       int M, int K, int N) {
  const int wave = blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  const int row0 = wave * R;
  if (row0 >= N) return;  // uniform per wave
  const int m0 = blockIdx.y * MR;
  const int nb = K / 256;
  const size_t row_bytes = (size_t)nb * 144;
  const int bl = lane >> 2, q = lane & 3;

  float acc[MR][R];
#pragma unroll
  for (int m = 0; m < MR; ++m)
#pragma unroll
    for (int r = 0; r < R; ++r) acc[m][r] = 0.f;

  for (int pass = 0; pass < nb; pass += 16) {
    const int b = pass + bl;
    if (b >= nb) continue;  // lane idles for the tail of a row
    // activations of this lane's 64 weights, and the two sub-block sums
    float xv[MR][64], xs1[MR], xs2[MR];
#pragma unroll
    for (int m = 0; m < MR; ++m) {
      const bool ok = m0 + m < M;
      const XT* xp = x + (size_t)(ok ? m0 + m : 0) * K + b * 256 + 64 * q;
      float s1 = 0.f, s2 = 0.f;
#pragma unroll
      for (int i = 0; i < 64; ++i) {
        xv[m][i] = ok ? to_f32(xp[i]) : 0.f;
        if (i < 32) s1 += xv[m][i]; else s2 += xv[m][i];
      }
      xs1[m] = s1;
      xs2[m] = s2;
    }
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const int n = row0 + r;
      if (n >= N) break;
      const uint8_t* blk = w + (size_t)n * row_bytes + (size_t)b * 144;
      const uint4 h = *reinterpret_cast<const uint4*>(blk);
      const uint4 c0 = *reinterpret_cast<const uint4*>(blk + 16 + 32 * q);
      const uint4 c1 = *reinterpret_cast<const uint4*>(blk + 32 + 32 * q);
      const Q4kScales s = q4k_scales(h, q);
      const uint32_t cw[8] = {c0.x, c0.y, c0.z, c0.w, c1.x, c1.y, c1.z, c1.w};
#pragma unroll
      for (int m = 0; m < MR; ++m) {
        float lo = 0.f, hi = 0.f;
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          const uint32_t l4 = cw[i] & 0x0F0F0F0Fu, h4 = (cw[i] >> 4) & 0x0F0F0F0Fu;
          lo = fmaf(xv[m][4 * i + 0], (float)(l4 & 0xFF), lo);
          lo = fmaf(xv[m][4 * i + 1], (float)((l4 >> 8) & 0xFF), lo);
          lo = fmaf(xv[m][4 * i + 2], (float)((l4 >> 16) & 0xFF), lo);
          lo = fmaf(xv[m][4 * i + 3], (float)(l4 >> 24), lo);
          hi = fmaf(xv[m][32 + 4 * i + 0], (float)(h4 & 0xFF), hi);
          hi = fmaf(xv[m][32 + 4 * i + 1], (float)((h4 >> 8) & 0xFF), hi);
          hi = fmaf(xv[m][32 + 4 * i + 2], (float)((h4 >> 16) & 0xFF), hi);
          hi = fmaf(xv[m][32 + 4 * i + 3], (float)(h4 >> 24), hi);
        }
        float t = s.d1 * lo - s.m1 * xs1[m];
        t = fmaf(s.d2, hi, t);
        t = fmaf(-s.m2, xs2[m], t);
        acc[m][r] += t;
      }
    }
  }
#pragma unroll
  for (int m = 0; m < MR; ++m)
#pragma unroll
    for (int r = 0; r < R; ++r) acc[m][r] = wave_sum(acc[m][r]);
  if (lane < R * MR) {
    // lane (m, r) writes row r of activation row m; select from registers without
    // dynamic indexing
    float v = 0.f;
    int mm = 0, rr = 0;
#pragma unroll
    for (int m = 0; m < MR; ++m)
#pragma unroll
      for (int r = 0; r < R; ++r)
        if (lane == m * R + r) { v = acc[m][r]; mm = m; rr = r; }
    const int n = row0 + rr;
    if (n < N && m0 + mm < M) {
      if (bias) v += bias[n];
      out[(size_t)(m0 + mm) * N + n] = from_f32<OT>(v);
    }
  }
}

template <int R, int MR, typename XT, typename OT>
static int launch_q4k(const void* x, const uint8_t* w, const float* bias, void* out, int M, int K, int N,
                      hipStream_t st) {
  const int waves = (N + R - 1) / R;
  dim3 grid((waves + 3) / 4, (M + MR - 1) / MR);
  hipLaunchKernelGGL((q4k_gemv_kernel<R, MR, XT, OT>), grid, dim3(256), 0, st, static_cast<const XT*>(x), w,
                     bias, static_cast<OT*>(out), M, K, N);
  return check_launch("q4k_gemv");
}

template <int MR>
static int q4k_types(const void* x, int xd, const uint8_t* w, const float* bias, void* out, int od, int M,
                     int K, int N, hipStream_t st) {
  constexpr int R = 4;
  if (xd == MIQ_F16) {
    if (od == MIQ_F16) return launch_q4k<R, MR, __half, __half>(x, w, bias, out, M, K, N, st);
    return launch_q4k<R, MR, __half, float>(x, w, bias, out, M, K, N, st);
  }
  if (od == MIQ_F16) return launch_q4k<R, MR, float, __half>(x, w, bias, out, M, K, N, st);
  return launch_q4k<R, MR, float, float>(x, w, bias, out, M, K, N, st);
}

}  // namespace miq

using namespace miq;

extern "C" int miq_q4k_dequant_f32(const uint8_t* blocks, float* out, int64_t n_blocks, void* stream) {
  MIQ_REQUIRE(n_blocks >= 0, MIQ_ERR_INVALID, "q4k_dequant_f32: n_blocks=%lld", (long long)n_blocks);
  if (n_blocks == 0) return MIQ_OK;
  MIQ_REQUIRE(blocks && out, MIQ_ERR_INVALID, "q4k_dequant_f32: null pointer");
  MIQ_REQUIRE(aligned(blocks, 16), MIQ_ERR_ALIGN, "q4k_dequant_f32: blocks must be 16-byte aligned");
  const int64_t threads = n_blocks * 4;
  hipLaunchKernelGGL(q4k_dequant_kernel, dim3((unsigned)((threads + 255) / 256)), dim3(256), 0,
                     static_cast<hipStream_t>(stream), blocks, out, n_blocks);
  return check_launch("q4k_dequant_f32");
}

extern "C" int miq_q4k_gemv(const void* x, int x_dtype, const uint8_t* w, const float* bias, void* out,
                            int out_dtype, int M, int K, int N, void* stream) {
  MIQ_REQUIRE(M >= 0 && K > 0 && N > 0, MIQ_ERR_INVALID, "q4k_gemv: M=%d K=%d N=%d", M, K, N);
  MIQ_REQUIRE(K % 256 == 0, MIQ_ERR_INVALID, "q4k_gemv: K=%d is not a multiple of 256", K);
  if (M == 0) return MIQ_OK;
  MIQ_REQUIRE(x && w && out, MIQ_ERR_INVALID, "q4k_gemv: null pointer");
  MIQ_REQUIRE(aligned(w, 16), MIQ_ERR_ALIGN, "q4k_gemv: weight must be 16-byte aligned");
  MIQ_REQUIRE(x_dtype == MIQ_F16 || x_dtype == MIQ_F32, MIQ_ERR_UNSUPPORTED, "q4k_gemv: x dtype");
  MIQ_REQUIRE(out_dtype == MIQ_F16 || out_dtype == MIQ_F32, MIQ_ERR_UNSUPPORTED, "q4k_gemv: out dtype");
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (M >= 2) return q4k_types<2>(x, x_dtype, w, bias, out, out_dtype, M, K, N, st);
  return q4k_types<1>(x, x_dtype, w, bias, out, out_dtype, M, K, N, st);
}
