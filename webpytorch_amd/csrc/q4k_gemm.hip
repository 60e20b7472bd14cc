// Q4_K prefill GEMM on the gfx950 matrix cores: out[m][n] = x[m][:] . W[n][:] (+ bias[n]) for
// many activation rows, W = N rows of K/256 Q4_K super-blocks as the file stores them.
//
// A Q4_K sub-block of 32 weights holds w = d1 c - m1 (d1 = d sc and m1 = dmin m: an fp16 scale
// times a 6-bit integer, exact in fp32; c the 4-bit code). Per sub-block
//   sum_k x_k w_k = d1 (sum_k x_k c_k) - m1 (sum_k x_k),
// with d1 = d sc, m1 = dmin m. The codes become fp16 B operands by OR-ing them into the
// mantissa of 1024.0 and subtracting 1024 (no conversion instruction per code), times sc; the
// row sums of x come precomputed per sub-block. The matrix cores do both sums (see gemm_kernel)
// and the accumulators take d and dmin once per super-block of 256 weights.
//
// fp32 activations enter as two fp16 rows each, hi = fp16(x 2^s) and lo = fp16(x 2^s - hi),
// with 2^s per row putting the row's largest |x| near 2^15 (s = 0 for rows holding NaN or Inf);
// the staging pass writes them and their sub-block sums as rows 2m and 2m + 1, and the GEMM's
// epilogue adds the pair and scales back. fp16 activations are staged as they are.
//
// Staged rows: xs[r][k] fp16, each 8-wide k block in the order (0, 2, 1, 3, 4, 6, 5, 7) that
// the code unpack produces (byte j of a code word holds value j in one nibble, and one
// v_and_or_b32 takes the nibbles of bytes 0 and 2, then of bytes 1 and 3); rs[r][k / 32] the
// sub-block sums of the staged fp16 values (fp32).
//
// Tiles: a workgroup of 4 waves computes 64 rows x 64 CG columns; wave w takes the CG groups of
// 16 columns from 16 CG w and all 64 rows (four 16-row MFMA tiles per group). K is walked one
// super-block (256 weights) at a time: the 64 x 256 activation tile sits in LDS (16-byte chunks
// XOR-swizzled by row, so the 16 rows that one operand read touches fall in different banks)
// and each lane holds its columns' super-block headers and 4 x 8 code bytes in registers.
// Workgroups are ordered XCD-major with row tiles fastest, so the row tiles of a column tile
// share that XCD's L2.
#include <math.h>

#include <type_traits>

#include "miq_common.h"

namespace miq {
namespace q4g {

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

// The low nibbles of 8 bytes (w0: bytes 0-3, w1: 4-7; the caller shifts the high nibbles down)
// as the fp16 B fragment, in the unpack's order.
__device__ __forceinline__ half8v b_codes(uint32_t w0, uint32_t w1) {
  const half2v k = (half2v){(_Float16)1024, (_Float16)1024};
  const half2v a = as_h2(and_or(w0, 0x000F000Fu, 0x64006400u)) - k;
  const half2v b = as_h2(and_or(w0 >> 8, 0x000F000Fu, 0x64006400u)) - k;
  const half2v c = as_h2(and_or(w1, 0x000F000Fu, 0x64006400u)) - k;
  const half2v d = as_h2(and_or(w1 >> 8, 0x000F000Fu, 0x64006400u)) - k;
  return (half8v){a[0], a[1], b[0], b[1], c[0], c[1], d[0], d[1]};
}

// y[r][n] for rows r < Mx of xs. Grid (ntiles * mtiles), 256 threads.
//
// Per super-block: P = sum_sb sc_sb (sum_k x_k c_k) on the fp16 matrix cores (the B operand is
// sc c, an integer below 1024, exact in fp16, so the eight sub-blocks chain in the MFMA
// accumulator), Q = sum_sb m_sb rs_sb on the fp32 matrix cores (two v_mfma_f32_16x16x4_f32:
// A the row sums, B the column's 6-bit mins), then acc += d P - dmin Q. The activation tile and
// the row sums arrive by LDS DMA into one of two buffers while the other is multiplied (the
// swizzle is applied on the source side: DMA lane l of a 1 KB block lands at slot l); each
// lane's super-block header and code bytes are loaded into registers one super-block ahead.
// The output (+ bias[n]) as OT. fp16 rows (PAIR false): y[row][n] = acc. fp32 rows (PAIR true):
// staged rows 2m and 2m + 1 are the hi and lo planes of row m, held by the same lane (rows
// 4 kb + r of a 16-row tile), so y[m][n] = (acc[2m] + acc[2m + 1]) 2^-s(m), s from rmax[m].
template <int CG, typename OT, bool PAIR>
__global__ __launch_bounds__(256) void gemm_kernel(const __half* __restrict__ xs, const float* __restrict__ rs,
                                                   const uint8_t* __restrict__ w, OT* __restrict__ y,
                                                   const float* __restrict__ bias, const float* __restrict__ rmax,
                                                   int Mx, int K, int N, int mtiles) {
  __shared__ __align__(16) __half at[2][kBM * 256];  // activation tiles, 16-byte chunks swizzled by row
  // sub-block sums [sub-block][row], rows of kRT floats: the lanes of one read take rows p and
  // sub-blocks kb, and at 64 floats (256 bytes) per sub-block the four kb share their banks
  constexpr int kRT = kBM + 16;
  __shared__ __align__(16) float rt[2][8 * kRT];
  const int T = (int)gridDim.x, L = (int)blockIdx.x;
  const int Lp = T % kXCDs == 0 ? (L % kXCDs) * (T / kXCDs) + L / kXCDs : L;
  const int mt = Lp % mtiles, nt = Lp / mtiles;
  const int m0 = mt * kBM, n0 = nt * 64 * CG;
  const int tid = threadIdx.x, lane = tid & 63, wave = uniform(tid >> 6), p = lane & 15, kb = lane >> 4;
  const int nsb = K / 256, K32 = K / 32;
  // wave w takes the column groups CG w .. CG w + CG - 1 (16 columns each); every operand read
  // of the activation tile feeds one MFMA per group
  int ncol[CG];
  const uint8_t* wr[CG];
#pragma unroll
  for (int c = 0; c < CG; ++c) {
    ncol[c] = n0 + 16 * (CG * wave + c) + p;
    const int n = min(ncol[c], N - 1);  // columns past N repeat the last one and are not stored
    wr[c] = w + (size_t)n * nsb * 144;
  }

  // this wave's share of the copies of super-block s into buffer b: 8 of the tile's 32 KB
  // (two rows per 1 KB block) and 2 of its 8 sub-block-sum columns
  auto issue = [&](int s, int b) __attribute__((always_inline)) {
    const uint32_t abase = lds_addr(at[b]), rbase = lds_addr(rt[b]);
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int j = wave * 8 + i, r = 2 * j + (lane >> 5), c = (lane & 31) ^ (r & 31);
      dma16(xs + (size_t)min(m0 + r, Mx - 1) * K + s * 256 + c * 8, uniform((int)(abase + j * 1024)));
    }
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const int sb = wave * 2 + i;
      dma4(rs + (size_t)min(m0 + lane, Mx - 1) * K32 + s * 8 + sb, uniform((int)(rbase + sb * kRT * 4)));
    }
  };
  uint4 hdr[CG], hdr_n[CG];
  uint2 cw[CG][4], cw_n[CG][4];
  auto load_b = [&](int s) __attribute__((always_inline)) {
#pragma unroll
    for (int c = 0; c < CG; ++c) {
      const uint8_t* bp = wr[c] + (size_t)s * 144;
      hdr_n[c] = *reinterpret_cast<const uint4*>(bp);
#pragma unroll
      for (int g = 0; g < 4; ++g) cw_n[c][g] = *reinterpret_cast<const uint2*>(bp + 16 + 32 * g + 8 * kb);
    }
  };

  float4v acc[CG][4];
#pragma unroll
  for (int c = 0; c < CG; ++c)
#pragma unroll
    for (int t = 0; t < 4; ++t) acc[c][t] = (float4v){0.f, 0.f, 0.f, 0.f};
  issue(0, 0);
  load_b(0);
  for (int s = 0; s < nsb; ++s) {
    wait_vmcnt<0>();  // this wave's copies of super-block s (and its header and codes) have landed
    __syncthreads();  // everyone's copies are in; everyone is done with the other buffer
    if (s + 1 < nsb) issue(s + 1, (s + 1) & 1);
#pragma unroll
    for (int c = 0; c < CG; ++c) {
      hdr[c] = hdr_n[c];
#pragma unroll
      for (int g = 0; g < 4; ++g) cw[c][g] = cw_n[c][g];
    }
    if (s + 1 < nsb) load_b(s + 1);
    const __half* a = at[s & 1];
    const float* r8 = rt[s & 1];
    float4v P[CG][4], Q[CG][4];
#pragma unroll
    for (int c = 0; c < CG; ++c)
#pragma unroll
      for (int t = 0; t < 4; ++t) P[c][t] = Q[c][t] = (float4v){0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int sb = 0; sb < 8; ++sb) {
      const int sh = 4 * (sb & 1);
      half8v bf[CG];
#pragma unroll
      for (int c = 0; c < CG; ++c) {
        uint32_t sc, mn;
        scale_min(hdr[c].y, hdr[c].z, hdr[c].w, sb, &sc, &mn);
        bf[c] = b_codes(cw[c][sb >> 1].x >> sh, cw[c][sb >> 1].y >> sh) * (_Float16)(float)sc;
      }
#pragma unroll
      for (int t = 0; t < 4; ++t) {
        const int r = 16 * t + p;
        const half8v af = *reinterpret_cast<const half8v*>(a + r * 256 + (((4 * sb + kb) ^ (r & 31)) * 8));
#pragma unroll
        for (int c = 0; c < CG; ++c) P[c][t] = __builtin_amdgcn_mfma_f32_16x16x32_f16(af, bf[c], P[c][t], 0, 0, 0);
      }
    }
    {  // Q = sum over the 8 sub-blocks of rs[row][sb] m[sb][col]: k = kb, then 4 + kb
      float m_lo[CG], m_hi[CG];
#pragma unroll
      for (int c = 0; c < CG; ++c) {
        uint32_t sc, mlo, mhi;
        scale_min(hdr[c].y, hdr[c].z, hdr[c].w, kb, &sc, &mlo);
        scale_min(hdr[c].y, hdr[c].z, hdr[c].w, 4 + kb, &sc, &mhi);
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
      const float d = __half2float(__ushort_as_half((unsigned short)(hdr[c].x & 0xFFFFu)));
      const float dmin = __half2float(__ushort_as_half((unsigned short)(hdr[c].x >> 16)));
#pragma unroll
      for (int t = 0; t < 4; ++t)
#pragma unroll
        for (int q = 0; q < 4; ++q) acc[c][t][q] = fmaf(d, P[c][t][q], fmaf(-dmin, Q[c][t][q], acc[c][t][q]));
    }
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


struct Ws {
  size_t xs, rs, rmax, bytes;
};
// workspace layout after the shared counter region: staged rows, sub-block sums, row maxima, y
static Ws layout(int M, int K, int N, int x_dtype) {
  const size_t R = x_dtype == MIQ_F32 ? 2 : 1, Mx = R * (size_t)M;
  auto up = [](size_t b) { return (b + 255) & ~(size_t)255; };
  Ws w;
  w.xs = kCounterBytes;
  w.rs = w.xs + up(Mx * K * 2);
  w.rmax = w.rs + up(Mx * (K / 32) * 4);
  w.bytes = w.rmax + up((size_t)M * 4);
  return w;
}

}  // namespace q4g
}  // namespace miq

using namespace miq;

extern "C" int miq_q4k_gemm_workspace(int M, int K, int N, int x_dtype, size_t* bytes) {
  MIQ_REQUIRE(bytes, MIQ_ERR_INVALID, "q4k_gemm_workspace: null output");
  MIQ_REQUIRE(M >= 0 && K > 0 && N > 0 && K % 256 == 0, MIQ_ERR_INVALID, "q4k_gemm_workspace: M=%d K=%d N=%d", M, K,
              N);
  MIQ_REQUIRE(x_dtype == MIQ_F16 || x_dtype == MIQ_F32, MIQ_ERR_UNSUPPORTED, "q4k_gemm_workspace: x dtype");
  *bytes = M == 0 ? 0 : q4g::layout(M, K, N, x_dtype).bytes;
  return MIQ_OK;
}

extern "C" int miq_q4k_gemm(const void* x, int x_dtype, const uint8_t* w, const float* bias, void* out, int out_dtype,
                            int M, int K, int N, void* workspace, size_t ws_bytes, void* stream) {
  MIQ_REQUIRE(M >= 0 && K > 0 && N > 0, MIQ_ERR_INVALID, "q4k_gemm: M=%d K=%d N=%d", M, K, N);
  MIQ_REQUIRE(K % 256 == 0, MIQ_ERR_INVALID, "q4k_gemm: K=%d is not a multiple of 256", K);
  MIQ_REQUIRE(x_dtype == MIQ_F16 || x_dtype == MIQ_F32, MIQ_ERR_UNSUPPORTED, "q4k_gemm: x dtype");
  MIQ_REQUIRE(out_dtype == MIQ_F16 || out_dtype == MIQ_F32, MIQ_ERR_UNSUPPORTED, "q4k_gemm: out dtype");
  if (M == 0) return MIQ_OK;
  MIQ_REQUIRE(x && w && out && workspace, MIQ_ERR_INVALID, "q4k_gemm: null pointer");
  MIQ_REQUIRE(aligned(w, 16) && aligned(x, 16) && aligned(workspace, 256), MIQ_ERR_ALIGN,
              "q4k_gemm: x and weight 16-byte, workspace 256-byte aligned");
  const q4g::Ws L = q4g::layout(M, K, N, x_dtype);
  MIQ_REQUIRE(ws_bytes >= L.bytes, MIQ_ERR_INVALID, "q4k_gemm: workspace %zu bytes, need %zu", ws_bytes, L.bytes);
  MIQ_REQUIRE(K <= 16384, MIQ_ERR_UNSUPPORTED, "q4k_gemm: K=%d too large to stage", K);
  hipStream_t st = static_cast<hipStream_t>(stream);
  unsigned char* b = static_cast<unsigned char*>(workspace);
  __half* xs = reinterpret_cast<__half*>(b + L.xs);
  float* rs = reinterpret_cast<float*>(b + L.rs);
  float* rmax = reinterpret_cast<float*>(b + L.rmax);
  const int R = x_dtype == MIQ_F32 ? 2 : 1, Mx = R * M;
  if (x_dtype == MIQ_F32) {
    if ((size_t)K * 4 > 64 * 1024) {
      const int rc = require_lds("q4k_gemm staging", (size_t)K * 4);
      if (rc) return rc;
    }
    hipLaunchKernelGGL(q4g::stage_kernel<float>, dim3(M), dim3(256), (size_t)K * 4, st, static_cast<const float*>(x), xs,
                       rs, rmax, K);
  } else {
    hipLaunchKernelGGL(q4g::stage_kernel<__half>, dim3(M), dim3(256), 0, st, static_cast<const __half*>(x), xs, rs, rmax,
                       K);
  }
  int rc = check_launch("q4k_gemm staging");
  if (rc) return rc;
  // two 16-column groups per wave (each activation operand read feeds two MFMAs) when that grid
  // still gives every CU two workgroups; otherwise one (measured at 4096 -> 14336: fp32 rows at
  // M = 512 288 -> 250 us, fp16 152 -> 149 us; at M = 64 the halved grid was slower, 36 -> 51 us)
  const int mtiles = (Mx + q4g::kBM - 1) / q4g::kBM;
  const long wide = (long)mtiles * ((N + 127) / 128);
  const dim3 grid((unsigned)(wide >= 2 * q4g::kCUs ? wide : mtiles * ((N + 63) / 64)));
  // the GEMM writes the output (+ bias) itself; fp32 rows add their hi/lo row pairs there
  auto gemm = [&](auto* dst, auto pair) {
    using OT = std::remove_pointer_t<decltype(dst)>;
    constexpr bool P = decltype(pair)::value;
    if (wide >= 2 * q4g::kCUs)
      hipLaunchKernelGGL((q4g::gemm_kernel<2, OT, P>), grid, dim3(256), 0, st, xs, rs, w, dst, bias, rmax, Mx, K, N,
                         mtiles);
    else
      hipLaunchKernelGGL((q4g::gemm_kernel<1, OT, P>), grid, dim3(256), 0, st, xs, rs, w, dst, bias, rmax, Mx, K, N,
                         mtiles);
    return check_launch("q4k_gemm");
  };
  if (R == 1) {
    if (out_dtype == MIQ_F16) return gemm(static_cast<__half*>(out), std::false_type{});
    return gemm(static_cast<float*>(out), std::false_type{});
  }
  if (out_dtype == MIQ_F16) return gemm(static_cast<__half*>(out), std::true_type{});
  return gemm(static_cast<float*>(out), std::true_type{});
}
