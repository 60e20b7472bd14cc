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
// with 16-byte loads; the lane reads its 64 activations from LDS once and walks R rows.
#include <type_traits>

#include "miq_common.h"

namespace miq {

constexpr int kQ4kDepth = 1;  // rows of a wave's blocks in flight ahead of the one computed (0: all)

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

// fp16 pair layout of a 64-wide code group in LDS: for code word wq (bytes 4wq..4wq+3) the
// 8 halves at 8wq are the pairs (4wq, 4wq+2), (4wq+1, 4wq+3) of the low sub-block and the same
// 32 further on for the high sub-block, matching nib_lo/nib_hi of the word and of the word
// shifted by 8.

// y[m][n] = sum_k x[m][k] * W[n][k] (+ bias[n]).
// A wave owns R consecutive rows per step (steps strided over the grid). Lane (slot, q) =
// (lane / 4, lane % 4) takes super-block p * 16 + slot of each row in pass p, and its 32-byte
// code group q: 64 weights of sub-blocks 2q (low nibbles) and 2q + 1 (high nibbles), at
// activations b * 256 + 64 q .. + 63. The workgroup stages x once in LDS (fp16 in the pair
// order of the nibble unpack, or fp32) with sums over each 32 activations; a lane reads its 64
// activations once per pass and reuses them for the R rows. The blocks of one row are issued
// ahead of the row computed (the first before x is staged): with every row of a wave in flight
// at once the arithmetic only starts when the memory phase is over, one row ahead lets it run
// under the loads of the next (4096 -> 14336: 13.1 -> 10.4 us with 8 rows a wave; 10.3 us with 7).
template <int R, int MR, typename XT, typename OT>
__global__ __launch_bounds__(256) void q4k_gemv_kernel(const XT* __restrict__ x, const uint8_t* __restrict__ w,
                                                       const float* __restrict__ bias, OT* __restrict__ out,
                                                       int M, int K, int N) {
  constexpr bool kHalf = std::is_same<XT, __half>::value;
  extern __shared__ __align__(16) unsigned char lds_raw[];
  // Each 64-value group of x sits in LDS with 16 bytes of padding after it (QG elements per
  // group): lane (slot, q) reads group 4 (pass 16 + slot) + q, and unpadded those groups lie
  // a multiple of 128 (fp16) or 256 (fp32) bytes apart, all on the same banks.
  constexpr int QG = kHalf ? 72 : 68;
  const int rowq = K / 64 * QG;  // elements per staged row
  _Float16* xs_h = reinterpret_cast<_Float16*>(lds_raw);
  float* xs_f = reinterpret_cast<float*>(lds_raw);
  float* xsum = reinterpret_cast<float*>(lds_raw + (size_t)MR * rowq * (kHalf ? 2 : 4));

  const int lane = threadIdx.x & 63;
  const int wave = uniform(threadIdx.x >> 6);
  const int m0 = blockIdx.y * MR;
  const int nb = K / 256;
  const size_t row_bytes = (size_t)nb * 144;
  const int slot = lane >> 2, q = lane & 3;
  const int groups = (N + R - 1) / R;
  const int wstride = gridDim.x * 4;
  int grp = blockIdx.x * 4 + wave;

  uint4 hd[R], c0[R], c1[R];
  // row r's block of a pass; the first D rows are issued ahead, row r + D when row r is computed
  constexpr int D = (kQ4kDepth > 0 && kQ4kDepth < R) ? kQ4kDepth : R;
  auto load_row = [&](int g, int pass, int r) __attribute__((always_inline)) {
    const int b = pass * 16 + slot;
    const int n = g * R + r;
    if (n < N && b < nb) {
      const uint8_t* blk = w + (size_t)n * row_bytes + (size_t)b * 144;
      hd[r] = *reinterpret_cast<const uint4*>(blk);
      c0[r] = *reinterpret_cast<const uint4*>(blk + 16 + 32 * q);
      c1[r] = *reinterpret_cast<const uint4*>(blk + 32 + 32 * q);
    }
  };
  auto load_rows = [&](int g, int pass) __attribute__((always_inline)) {
#pragma unroll
    for (int r = 0; r < D; ++r) load_row(g, pass, r);
  };
  auto load_ahead = [&](int g, int pass, int r) __attribute__((always_inline)) {
    if constexpr (D < R) {
      if (r + D < R) {
        __builtin_amdgcn_sched_barrier(0);
        load_row(g, pass, r + D);
        __builtin_amdgcn_sched_barrier(0);
      }
    }
  };
  if (grp < groups) load_rows(grp, 0);

  // ---- stage x and its 32-wide sums ----
  // 8 consecutive activations per thread and step; 4 threads make one 32-wide sum
  for (int ci = threadIdx.x; ci < MR * K / 8; ci += 256) {
    const int m = ci / (K / 8), k = (ci - m * (K / 8)) * 8;
    float v[8];
    if (m0 + m < M) {
      load8(x + (size_t)(m0 + m) * K + k, v);
    } else {
#pragma unroll
      for (int j = 0; j < 8; ++j) v[j] = 0.f;
    }
    float sum = ((v[0] + v[1]) + (v[2] + v[3])) + ((v[4] + v[5]) + (v[6] + v[7]));
    sum = quad_sum(sum);
    if ((lane & 3) == 0) xsum[m * (K / 32) + k / 32] = sum;
    if constexpr (kHalf) {
      // activations c0..c0+7 of a 64-wide group land in code words wq and wq+1 (wq = (c0 % 32) / 4)
      // at slots 4h..4h+3 (h = c0 / 32), in the order (x0, x2, x1, x3)
      const int c0 = k & 63, h = c0 >> 5, wq = (c0 & 31) >> 2;
      _Float16* base = xs_h + (size_t)m * rowq + (k >> 6) * QG + wq * 8 + h * 4;
      *reinterpret_cast<uint2*>(base) = make_uint2(pack_h2(v[0], v[2]), pack_h2(v[1], v[3]));
      *reinterpret_cast<uint2*>(base + 8) = make_uint2(pack_h2(v[4], v[6]), pack_h2(v[5], v[7]));
    } else {
      float4* d = reinterpret_cast<float4*>(xs_f + (size_t)m * rowq + (k >> 6) * QG + (k & 63));
      d[0] = make_float4(v[0], v[1], v[2], v[3]);
      d[1] = make_float4(v[4], v[5], v[6], v[7]);
    }
  }
  __syncthreads();

  const int passes = (nb + 15) / 16;
  for (; grp < groups; grp += wstride) {
    float acc[MR][R];
#pragma unroll
    for (int m = 0; m < MR; ++m)
#pragma unroll
      for (int r = 0; r < R; ++r) acc[m][r] = 0.f;
    for (int pass = 0; pass < passes; ++pass) {
      if (pass > 0) load_rows(grp, pass);
      const int b = pass * 16 + slot;
      if (b < nb) {
        const int kb = b * 256 + 64 * q;
#pragma unroll
        for (int m = 0; m < MR; ++m) {
          const float sA = xsum[m * (K / 32) + kb / 32], sB = xsum[m * (K / 32) + kb / 32 + 1];
          if constexpr (kHalf) {
            half2v xv[8][4];
            const uint4* xp = reinterpret_cast<const uint4*>(xs_h + (size_t)m * rowq + (kb >> 6) * QG);
#pragma unroll
            for (int wq = 0; wq < 8; ++wq) {
              const uint4 t = xp[wq];
              xv[wq][0] = as_h2(t.x); xv[wq][1] = as_h2(t.y); xv[wq][2] = as_h2(t.z); xv[wq][3] = as_h2(t.w);
            }
#pragma unroll
            for (int r = 0; r < R; ++r) {
              const int n = grp * R + r;
              if (m == 0) load_ahead(grp, pass, r);
              if (n >= N) break;
              uint4 h4 = hd[r];
              uint32_t cw[8] = {c0[r].x, c0[r].y, c0[r].z, c0[r].w, c1[r].x, c1[r].y, c1[r].z, c1[r].w};
              // An empty asm that takes this row's words and the previous row's sum keeps the rows
              // in order (otherwise every row is unpacked at once and the registers run out).
              asm volatile("" : "+v"(cw[0]), "+v"(cw[1]), "+v"(cw[2]), "+v"(cw[3]), "+v"(cw[4]), "+v"(cw[5]),
                           "+v"(cw[6]), "+v"(cw[7]), "+v"(h4.x), "+v"(h4.y), "+v"(h4.z), "+v"(h4.w),
                           "+v"(acc[m][r > 0 ? r - 1 : 0]));
              const Q4kScales s = q4k_scales(h4, q);
              float pa = 0.f, pb = 0.f;
#pragma unroll
              for (int wq = 0; wq < 8; ++wq) {
                const uint32_t v0 = cw[wq], v8 = cw[wq] >> 8;
                pa = dot2(xv[wq][0], nib_lo(v0), pa);
                pa = dot2(xv[wq][1], nib_lo(v8), pa);
                pb = dot2(xv[wq][2], nib_hi(v0), pb);
                pb = dot2(xv[wq][3], nib_hi(v8), pb);
              }
              float t = fmaf(s.d1, pa, -s.m1 * sA);
              t = fmaf(s.d2, pb, t);
              acc[m][r] += fmaf(-s.m2, sB, t);
            }
          } else {
            const float* xf = xs_f + (size_t)m * rowq + (kb >> 6) * QG;
#pragma unroll
            for (int r = 0; r < R; ++r) {
              const int n = grp * R + r;
              if (m == 0) load_ahead(grp, pass, r);
              if (n >= N) break;
              uint4 h4 = hd[r];
              uint32_t cw[8] = {c0[r].x, c0[r].y, c0[r].z, c0[r].w, c1[r].x, c1[r].y, c1[r].z, c1[r].w};
              // An empty asm that takes this row's words and the previous row's sum keeps the rows
              // in order (otherwise every row is unpacked at once and the registers run out).
              asm volatile("" : "+v"(cw[0]), "+v"(cw[1]), "+v"(cw[2]), "+v"(cw[3]), "+v"(cw[4]), "+v"(cw[5]),
                           "+v"(cw[6]), "+v"(cw[7]), "+v"(h4.x), "+v"(h4.y), "+v"(h4.z), "+v"(h4.w),
                           "+v"(acc[m][r > 0 ? r - 1 : 0]));
              const Q4kScales s = q4k_scales(h4, q);
              float pa = 0.f, pb = 0.f;
#pragma unroll
              for (int wq = 0; wq < 8; ++wq) {
                const float4 xa = *reinterpret_cast<const float4*>(xf + 4 * wq);
                const float4 xb = *reinterpret_cast<const float4*>(xf + 32 + 4 * wq);
                const uint32_t l4 = cw[wq] & 0x0F0F0F0Fu, h4 = (cw[wq] >> 4) & 0x0F0F0F0Fu;
                pa = fmaf(xa.x, (float)(l4 & 0xFF), pa);
                pa = fmaf(xa.y, (float)((l4 >> 8) & 0xFF), pa);
                pa = fmaf(xa.z, (float)((l4 >> 16) & 0xFF), pa);
                pa = fmaf(xa.w, (float)(l4 >> 24), pa);
                pb = fmaf(xb.x, (float)(h4 & 0xFF), pb);
                pb = fmaf(xb.y, (float)((h4 >> 8) & 0xFF), pb);
                pb = fmaf(xb.z, (float)((h4 >> 16) & 0xFF), pb);
                pb = fmaf(xb.w, (float)(h4 >> 24), pb);
              }
              float t = fmaf(s.d1, pa, -s.m1 * sA);
              t = fmaf(s.d2, pb, t);
              acc[m][r] += fmaf(-s.m2, sB, t);
            }
          }
        }
      }
    }
#pragma unroll
    for (int m = 0; m < MR; ++m)
#pragma unroll
      for (int r = 0; r < R; ++r) acc[m][r] = wave_sum(acc[m][r]);
    if (lane < R * MR) {
      // lane (m, r) writes row r of activation row m; registers selected without dynamic indexing
      float v = 0.f;
      int mm = 0, rr = 0;
#pragma unroll
      for (int m = 0; m < MR; ++m)
#pragma unroll
        for (int r = 0; r < R; ++r)
          if (lane == m * R + r) { v = acc[m][r]; mm = m; rr = r; }
      const int n = grp * R + rr;
      if (n < N && m0 + mm < M) {
        if (bias) v += bias[n];
        out[(size_t)(m0 + mm) * N + n] = from_f32<OT>(v);
      }
    }
    if (grp + wstride < groups) load_rows(grp + wstride, 0);
  }
}

template <int R, int MR, typename XT, typename OT>
static int launch_q4k(const void* x, const uint8_t* w, const float* bias, void* out, int M, int K, int N,
                      hipStream_t st) {
  auto kern = q4k_gemv_kernel<R, MR, XT, OT>;
  const size_t lds = (size_t)MR * (K / 64) * (std::is_same<XT, __half>::value ? 144 : 272) + (size_t)MR * (K / 32) * 4;
  MIQ_REQUIRE(lds <= 160 * 1024, MIQ_ERR_UNSUPPORTED, "q4k_gemv: K=%d too large to stage", K);
  if (lds > 64 * 1024) {
    const int rc = require_lds("q4k_gemv", lds);
    if (rc) return rc;
  }
  const int groups = (N + R - 1) / R;
  int wgs = (groups + 3) / 4;
  if (wgs > 4 * kCUs) wgs = 4 * kCUs;
  dim3 grid(wgs, (M + MR - 1) / MR);
  hipLaunchKernelGGL(kern, grid, dim3(256), lds, st, static_cast<const XT*>(x), w, bias,
                     static_cast<OT*>(out), M, K, N);
  return check_launch("q4k_gemv");
}

template <int R, int MR>
static int q4k_types(const void* x, int xd, const uint8_t* w, const float* bias, void* out, int od, int M,
                     int K, int N, hipStream_t st) {
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
  MIQ_REQUIRE(aligned(w, 16) && aligned(x, 16), MIQ_ERR_ALIGN, "q4k_gemv: x and weight must be 16-byte aligned");
  MIQ_REQUIRE(x_dtype == MIQ_F16 || x_dtype == MIQ_F32, MIQ_ERR_UNSUPPORTED, "q4k_gemv: x dtype");
  MIQ_REQUIRE(out_dtype == MIQ_F16 || out_dtype == MIQ_F32, MIQ_ERR_UNSUPPORTED, "q4k_gemv: out dtype");
  hipStream_t st = static_cast<hipStream_t>(stream);
  // Rows per wave: 8, or 7 where that gives the busiest CU fewer rows (its workgroups, four
  // waves each, rounded up over the CUs): 4096 -> 14336 is 448 workgroups at 8 rows (two on
  // most CUs, one on the rest) but 512 at 7, two on every CU.
  auto busiest = [&](int R) { return R * (((N + R - 1) / R + 4 * kCUs - 1) / (4 * kCUs)); };
  if (busiest(7) < busiest(8)) {
    if (M >= 2) return q4k_types<7, 2>(x, x_dtype, w, bias, out, out_dtype, M, K, N, st);
    return q4k_types<7, 1>(x, x_dtype, w, bias, out, out_dtype, M, K, N, st);
  }
  if (M >= 2) return q4k_types<8, 2>(x, x_dtype, w, bias, out, out_dtype, M, K, N, st);
  return q4k_types<8, 1>(x, x_dtype, w, bias, out, out_dtype, M, K, N, st);
}
