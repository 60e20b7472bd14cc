// GPTQ int4/int8 dequant and decode GEMV for gfx950.
//
// Weight layout (AutoGPTQ, unchanged from disk): qweight int32 [K/per][N], per = 32/bits,
// code of row k in bits ((k % per) * bits); qzeros int32 [K/gs][N/per] packed along N;
// scales fp16 or fp32 [K/gs][N]. W[k][n] = s[g][n] * (q[k][n] - (z[g][n] + zero_offset)).
//
// GEMV mapping: one lane owns 4 adjacent columns and reads them with one 16-byte load per
// packed row (a wave reads 1 KB contiguous per row). The waves of a workgroup split K into
// contiguous chunks of CK activations; the workgroup reduces its waves' partial sums in a
// fixed order through LDS, so results are deterministic. Activations (optionally gathered
// through an act-order permutation) are staged once per workgroup in LDS as fp32, with
// per-chunk sums so the zero point is applied once per chunk: sum x*(q - z) is computed as
// sum x*q - z * sum x.
#include "miq_common.h"

namespace miq {

// ------------------------------------------------------------------------------------
// fp32 dequant: one thread per (packed row, column); bit-exact with the float64 product
// rounded once to float32 for integer zero offsets.
template <int BITS, typename ST>
__global__ __launch_bounds__(256) void gptq_dequant_kernel(
    const uint32_t* __restrict__ qw, const uint32_t* __restrict__ qz, const ST* __restrict__ sc,
    const int32_t* __restrict__ g_idx, float* __restrict__ out, int K, int N, int gs, float zoff) {
  constexpr int PER = 32 / BITS;
  constexpr uint32_t MASK = (1u << BITS) - 1u;
  const int n = blockIdx.x * blockDim.x + threadIdx.x;
  const int r = blockIdx.y;
  if (n >= N) return;
  const uint32_t w = qw[(size_t)r * N + n];
  const int NZ = N / PER;
#pragma unroll
  for (int j = 0; j < PER; ++j) {
    const int k = r * PER + j;
    const int g = g_idx ? g_idx[k] : k / gs;
    const uint32_t z = (qz[(size_t)g * NZ + n / PER] >> ((n % PER) * BITS)) & MASK;
    const float s = to_f32(sc[(size_t)g * N + n]);
    const float q = (float)((w >> (j * BITS)) & MASK);
    out[(size_t)k * N + n] = s * (q - ((float)z + zoff));
  }
}

// ------------------------------------------------------------------------------------
// Act-order repack: qweight rows reordered so that packed row r holds original rows
// perm[r*per .. r*per+per-1]; a thread builds one output word.
template <int BITS>
__global__ __launch_bounds__(256) void gptq_repack_kernel(const uint32_t* __restrict__ qw,
                                                          const int32_t* __restrict__ perm,
                                                          uint32_t* __restrict__ out, int K, int N) {
  constexpr int PER = 32 / BITS;
  constexpr uint32_t MASK = (1u << BITS) - 1u;
  const int n = blockIdx.x * blockDim.x + threadIdx.x;
  const int r = blockIdx.y;
  if (n >= N) return;
  uint32_t w = 0;
#pragma unroll
  for (int j = 0; j < PER; ++j) {
    const int k = perm[r * PER + j];
    const uint32_t q = (qw[(size_t)(k / PER) * N + n] >> ((k % PER) * BITS)) & MASK;
    w |= q << (j * BITS);
  }
  out[(size_t)r * N + n] = w;
}

// ------------------------------------------------------------------------------------
// GEMV / skinny GEMM (M <= 8).
template <int BITS> struct Unpack;

// int4: one word = 8 consecutive rows of one column.
template <> struct Unpack<4> {
  static constexpr int PER = 8;
  // part += sum_j x[j] * code_j  for the 8 rows held in w
  __device__ __forceinline__ static float dot(uint32_t w, const float* x, float part) {
    const uint32_t lo = w & 0x0F0F0F0Fu;         // codes of rows 0,2,4,6
    const uint32_t hi = (w >> 4) & 0x0F0F0F0Fu;  // codes of rows 1,3,5,7
    part = fmaf(x[0], (float)(lo & 0xFFu), part);
    part = fmaf(x[1], (float)(hi & 0xFFu), part);
    part = fmaf(x[2], (float)((lo >> 8) & 0xFFu), part);
    part = fmaf(x[3], (float)((hi >> 8) & 0xFFu), part);
    part = fmaf(x[4], (float)((lo >> 16) & 0xFFu), part);
    part = fmaf(x[5], (float)((hi >> 16) & 0xFFu), part);
    part = fmaf(x[6], (float)(lo >> 24), part);
    part = fmaf(x[7], (float)(hi >> 24), part);
    return part;
  }
};

// int8: one word = 4 consecutive rows of one column.
template <> struct Unpack<8> {
  static constexpr int PER = 4;
  __device__ __forceinline__ static float dot(uint32_t w, const float* x, float part) {
    part = fmaf(x[0], (float)(w & 0xFFu), part);
    part = fmaf(x[1], (float)((w >> 8) & 0xFFu), part);
    part = fmaf(x[2], (float)((w >> 16) & 0xFFu), part);
    part = fmaf(x[3], (float)(w >> 24), part);
    return part;
  }
};

template <typename ST> __device__ __forceinline__ void load4(const ST* p, float* v);
template <> __device__ __forceinline__ void load4<float>(const float* p, float* v) {
  const float4 t = *reinterpret_cast<const float4*>(p);
  v[0] = t.x; v[1] = t.y; v[2] = t.z; v[3] = t.w;
}
template <> __device__ __forceinline__ void load4<__half>(const __half* p, float* v) {
  const uint2 t = *reinterpret_cast<const uint2*>(p);
  v[0] = __half2float(__ushort_as_half((unsigned short)(t.x & 0xFFFF)));
  v[1] = __half2float(__ushort_as_half((unsigned short)(t.x >> 16)));
  v[2] = __half2float(__ushort_as_half((unsigned short)(t.y & 0xFFFF)));
  v[3] = __half2float(__ushort_as_half((unsigned short)(t.y >> 16)));
}

// LDS: xs[MR][K] fp32 activations, then xsum[MR][K/CK] chunk sums. Re-used for the
// cross-wave reduction, red[S][MR][256].
// At most 32 / MR waves per workgroup (the reduction buffer is S * MR KB), which bounds the
// workgroup size and so the register budget per lane.
template <int MR> constexpr int gemv_threads() { return MR >= 8 ? 256 : (MR >= 4 ? 512 : 1024); }

template <int BITS, int MR, int CK, typename XT, typename ST, typename OT>
__global__ __launch_bounds__(gemv_threads<MR>()) void gptq_gemv_kernel(
    const XT* __restrict__ x, const int32_t* __restrict__ perm, const uint32_t* __restrict__ qw,
    const uint32_t* __restrict__ qz, const ST* __restrict__ sc, const float* __restrict__ bias,
    OT* __restrict__ out, int M, int K, int N, int gs, float zoff) {
  constexpr int PER = Unpack<BITS>::PER;
  constexpr int RPC = CK / PER;  // packed rows per chunk
  constexpr uint32_t MASK = (1u << BITS) - 1u;
  extern __shared__ float lds[];
  float* xs = lds;
  const int NC = K / CK;
  float* xsum = lds + MR * K;

  const int S = blockDim.x >> 6;
  const int wave = uniform(threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  const int m0 = blockIdx.y * MR;

  // ---- stage activations (gathered through perm for act-order) ----
  for (int i = threadIdx.x; i < MR * K; i += blockDim.x) {
    const int m = i / K, k = i - m * K;
    const int src = perm ? perm[k] : k;
    xs[i] = (m0 + m < M) ? to_f32(x[(size_t)(m0 + m) * K + src]) : 0.f;
  }
  __syncthreads();
  for (int it = wave; it < MR * NC; it += S) {
    const float* p = xs + (it / NC) * K + (it % NC) * CK;
    float s = 0.f;
    for (int j = lane; j < CK; j += 64) s += p[j];
    s = wave_sum(s);
    if (lane == 0) xsum[it] = s;
  }
  __syncthreads();

  const int n0 = (blockIdx.x * 64 + lane) * 4;
  const int c0 = wave * NC / S, c1 = (wave + 1) * NC / S;
  float acc[MR][4];
#pragma unroll
  for (int m = 0; m < MR; ++m)
#pragma unroll
    for (int c = 0; c < 4; ++c) acc[m][c] = 0.f;

  if (n0 < N && c0 < c1) {
    const int NZ = N / PER;
    int g = -1;
    float s4[4], z4[4], part[MR][4], xg[MR];
    for (int ch = c0; ch < c1; ++ch) {
      const int k0 = ch * CK;
      const int gc = k0 / gs;
      if (gc != g) {
        if (g >= 0) {
#pragma unroll
          for (int m = 0; m < MR; ++m)
#pragma unroll
            for (int c = 0; c < 4; ++c) acc[m][c] = fmaf(s4[c], part[m][c] - z4[c] * xg[m], acc[m][c]);
        }
        g = gc;
        load4<ST>(sc + (size_t)g * N + n0, s4);
        const uint32_t zw = qz[(size_t)g * NZ + n0 / PER] >> ((n0 % PER) * BITS);
#pragma unroll
        for (int c = 0; c < 4; ++c) z4[c] = (float)((zw >> (c * BITS)) & MASK) + zoff;
#pragma unroll
        for (int m = 0; m < MR; ++m) {
          xg[m] = 0.f;
#pragma unroll
          for (int c = 0; c < 4; ++c) part[m][c] = 0.f;
        }
      }
      // all loads of the chunk first, then the math
      uint4 w[RPC];
      const uint32_t* base = qw + (size_t)(k0 / PER) * N + n0;
#pragma unroll
      for (int r = 0; r < RPC; ++r) w[r] = *reinterpret_cast<const uint4*>(base + (size_t)r * N);
#pragma unroll
      for (int m = 0; m < MR; ++m) {
        xg[m] += xsum[m * NC + ch];
        const float* xr = xs + m * K + k0;
#pragma unroll
        for (int r = 0; r < RPC; ++r) {
          float xv[PER];
#pragma unroll
          for (int j = 0; j < PER; j += 4) {
            const float4 t = *reinterpret_cast<const float4*>(xr + r * PER + j);
            xv[j] = t.x; xv[j + 1] = t.y; xv[j + 2] = t.z; xv[j + 3] = t.w;
          }
          part[m][0] = Unpack<BITS>::dot(w[r].x, xv, part[m][0]);
          part[m][1] = Unpack<BITS>::dot(w[r].y, xv, part[m][1]);
          part[m][2] = Unpack<BITS>::dot(w[r].z, xv, part[m][2]);
          part[m][3] = Unpack<BITS>::dot(w[r].w, xv, part[m][3]);
        }
      }
    }
#pragma unroll
    for (int m = 0; m < MR; ++m)
#pragma unroll
      for (int c = 0; c < 4; ++c) acc[m][c] = fmaf(s4[c], part[m][c] - z4[c] * xg[m], acc[m][c]);
  }

  // ---- deterministic cross-wave reduction ----
  __syncthreads();
  float* red = lds;  // [S][MR][256]
#pragma unroll
  for (int m = 0; m < MR; ++m)
#pragma unroll
    for (int c = 0; c < 4; ++c) red[(wave * MR + m) * 256 + lane * 4 + c] = acc[m][c];
  __syncthreads();
  for (int i = threadIdx.x; i < MR * 256; i += blockDim.x) {
    const int m = i >> 8, q = i & 255;
    const int n = blockIdx.x * 256 + q;
    if (m0 + m >= M || n >= N) continue;
    float s = 0.f;
    for (int w = 0; w < S; ++w) s += red[(w * MR + m) * 256 + q];
    if (bias) s += bias[n];
    out[(size_t)(m0 + m) * N + n] = from_f32<OT>(s);
  }
}

// ------------------------------------------------------------------------------------
template <int BITS, int MR, int CK, typename XT, typename ST, typename OT>
static int launch_gemv(const void* x, const int32_t* perm, const int32_t* qw, const int32_t* qz,
                       const void* sc, const float* bias, void* out, int M, int K, int N, int gs,
                       float zoff, hipStream_t st) {
  const int tiles = (N + 255) / 256;
  const int NC = K / CK;
  // Waves per workgroup: enough workgroups x waves to fill 256 CUs several times, no more
  // waves than chunks, and a reduction buffer that fits beside the staged activations.
  int S = (8 * kCUs + tiles - 1) / tiles;
  S = S < 1 ? 1 : S;
  S = S > 16 ? 16 : S;
  S = S > NC ? NC : S;
  while (S > 1 && 64 * S > gemv_threads<MR>()) --S;
  size_t stage = (size_t)MR * K * 4 + (size_t)MR * NC * 4;
  size_t redb = (size_t)S * MR * 256 * 4;
  size_t lds = stage > redb ? stage : redb;
  MIQ_REQUIRE(lds <= 160 * 1024, MIQ_ERR_UNSUPPORTED, "gptq_gemv: K=%d too large for one LDS stage", K);
  auto kern = gptq_gemv_kernel<BITS, MR, CK, XT, ST, OT>;
  if (lds > 64 * 1024) {
    static bool raised = false;  // once per instantiation: allow up to the 160 KB of gfx950 LDS
    if (!raised) {
      hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(kern),
                                         hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024);
      MIQ_REQUIRE(e == hipSuccess, MIQ_ERR_HIP, "gptq_gemv: LDS attribute: %s", hipGetErrorString(e));
      raised = true;
    }
  }
  dim3 grid(tiles, (M + MR - 1) / MR);
  hipLaunchKernelGGL(kern, grid, dim3(64 * S), lds, st,
                     static_cast<const XT*>(x), perm, reinterpret_cast<const uint32_t*>(qw),
                     reinterpret_cast<const uint32_t*>(qz), static_cast<const ST*>(sc), bias,
                     static_cast<OT*>(out), M, K, N, gs, zoff);
  return check_launch("gptq_gemv");
}

template <int BITS, int MR, int CK>
static int gemv_types(const void* x, int xd, const int32_t* perm, const int32_t* qw, const int32_t* qz,
                      const void* sc, int sd, const float* bias, void* out, int od, int M, int K, int N,
                      int gs, float zoff, hipStream_t st) {
#define MIQ_GEMV_CASE(XT, ST, OT)                                                                   \
  return launch_gemv<BITS, MR, CK, XT, ST, OT>(x, perm, qw, qz, sc, bias, out, M, K, N, gs, zoff, st)
  if (xd == MIQ_F16) {
    if (sd == MIQ_F16) { if (od == MIQ_F16) MIQ_GEMV_CASE(__half, __half, __half); MIQ_GEMV_CASE(__half, __half, float); }
    if (od == MIQ_F16) MIQ_GEMV_CASE(__half, float, __half);
    MIQ_GEMV_CASE(__half, float, float);
  }
  if (sd == MIQ_F16) { if (od == MIQ_F16) MIQ_GEMV_CASE(float, __half, __half); MIQ_GEMV_CASE(float, __half, float); }
  if (od == MIQ_F16) MIQ_GEMV_CASE(float, float, __half);
  MIQ_GEMV_CASE(float, float, float);
#undef MIQ_GEMV_CASE
}

template <int BITS, int CK>
static int gemv_mr(const void* x, int xd, const int32_t* perm, const int32_t* qw, const int32_t* qz,
                   const void* sc, int sd, const float* bias, void* out, int od, int M, int K, int N,
                   int gs, float zoff, hipStream_t st) {
  // rows of x per workgroup; the activation stage must fit LDS
  if (M >= 8 && (size_t)8 * K * 4 <= 64 * 1024)
    return gemv_types<BITS, 8, CK>(x, xd, perm, qw, qz, sc, sd, bias, out, od, M, K, N, gs, zoff, st);
  if (M >= 4 && (size_t)4 * K * 4 <= 96 * 1024)
    return gemv_types<BITS, 4, CK>(x, xd, perm, qw, qz, sc, sd, bias, out, od, M, K, N, gs, zoff, st);
  if (M >= 2 && (size_t)2 * K * 4 <= 128 * 1024)
    return gemv_types<BITS, 2, CK>(x, xd, perm, qw, qz, sc, sd, bias, out, od, M, K, N, gs, zoff, st);
  return gemv_types<BITS, 1, CK>(x, xd, perm, qw, qz, sc, sd, bias, out, od, M, K, N, gs, zoff, st);
}

int check_gptq_dims(const char* who, int K, int N, int gs, int bits) {
  MIQ_REQUIRE(bits == 4 || bits == 8, MIQ_ERR_UNSUPPORTED, "%s: bits=%d (only 4 and 8)", who, bits);
  const int per = 32 / bits;
  MIQ_REQUIRE(K > 0 && N > 0 && gs > 0, MIQ_ERR_INVALID, "%s: K=%d N=%d gs=%d must be positive", who, K, N, gs);
  MIQ_REQUIRE(K % gs == 0 && K % per == 0 && N % per == 0, MIQ_ERR_INVALID,
              "%s: dims must divide group/pack size (K=%d N=%d gs=%d bits=%d)", who, K, N, gs, bits);
  return MIQ_OK;
}

}  // namespace miq

using namespace miq;

extern "C" int miq_gptq_dequant_f32(const int32_t* qweight, const int32_t* qzeros, const void* scales,
                                    int scales_dtype, const int32_t* g_idx, float* out, int K, int N,
                                    int gs, int bits, float zero_offset, void* stream) {
  int rc = check_gptq_dims("gptq_dequant_f32", K, N, gs, bits);
  if (rc) return rc;
  MIQ_REQUIRE(qweight && qzeros && scales && out, MIQ_ERR_INVALID, "gptq_dequant_f32: null pointer");
  hipStream_t st = static_cast<hipStream_t>(stream);
  dim3 grid((N + 255) / 256, K / (32 / bits));
  const uint32_t* qw = reinterpret_cast<const uint32_t*>(qweight);
  const uint32_t* qz = reinterpret_cast<const uint32_t*>(qzeros);
  if (bits == 4) {
    if (scales_dtype == MIQ_F16)
      hipLaunchKernelGGL((gptq_dequant_kernel<4, __half>), grid, dim3(256), 0, st, qw, qz,
                         static_cast<const __half*>(scales), g_idx, out, K, N, gs, zero_offset);
    else
      hipLaunchKernelGGL((gptq_dequant_kernel<4, float>), grid, dim3(256), 0, st, qw, qz,
                         static_cast<const float*>(scales), g_idx, out, K, N, gs, zero_offset);
  } else {
    if (scales_dtype == MIQ_F16)
      hipLaunchKernelGGL((gptq_dequant_kernel<8, __half>), grid, dim3(256), 0, st, qw, qz,
                         static_cast<const __half*>(scales), g_idx, out, K, N, gs, zero_offset);
    else
      hipLaunchKernelGGL((gptq_dequant_kernel<8, float>), grid, dim3(256), 0, st, qw, qz,
                         static_cast<const float*>(scales), g_idx, out, K, N, gs, zero_offset);
  }
  return check_launch("gptq_dequant_f32");
}

extern "C" int miq_gptq_repack_rows(const int32_t* qweight, const int32_t* perm, int32_t* out, int K,
                                    int N, int bits, void* stream) {
  MIQ_REQUIRE(bits == 4 || bits == 8, MIQ_ERR_UNSUPPORTED, "gptq_repack_rows: bits=%d", bits);
  MIQ_REQUIRE(K > 0 && N > 0 && K % (32 / bits) == 0, MIQ_ERR_INVALID, "gptq_repack_rows: K=%d N=%d", K, N);
  MIQ_REQUIRE(qweight && perm && out && (const void*)qweight != (const void*)out, MIQ_ERR_INVALID,
              "gptq_repack_rows: null or aliased pointer");
  dim3 grid((N + 255) / 256, K / (32 / bits));
  hipStream_t st = static_cast<hipStream_t>(stream);
  const uint32_t* qw = reinterpret_cast<const uint32_t*>(qweight);
  uint32_t* o = reinterpret_cast<uint32_t*>(out);
  if (bits == 4)
    hipLaunchKernelGGL((gptq_repack_kernel<4>), grid, dim3(256), 0, st, qw, perm, o, K, N);
  else
    hipLaunchKernelGGL((gptq_repack_kernel<8>), grid, dim3(256), 0, st, qw, perm, o, K, N);
  return check_launch("gptq_repack_rows");
}

extern "C" int miq_gptq_gemv(const void* x, int x_dtype, const int32_t* perm, const int32_t* qweight,
                             const int32_t* qzeros, const void* scales, int scales_dtype, const float* bias,
                             void* out, int out_dtype, int M, int K, int N, int gs, int bits,
                             float zero_offset, void* stream) {
  int rc = check_gptq_dims("gptq_gemv", K, N, gs, bits);
  if (rc) return rc;
  MIQ_REQUIRE(M >= 0, MIQ_ERR_INVALID, "gptq_gemv: M=%d", M);
  if (M == 0) return MIQ_OK;
  MIQ_REQUIRE(x && qweight && qzeros && scales && out, MIQ_ERR_INVALID, "gptq_gemv: null pointer");
  MIQ_REQUIRE(N % 4 == 0 && aligned(qweight, 16) && aligned(scales, scales_dtype == MIQ_F16 ? 8 : 16),
              MIQ_ERR_ALIGN, "gptq_gemv: qweight must be 16-byte aligned and N %% 4 == 0");
  MIQ_REQUIRE(x_dtype == MIQ_F16 || x_dtype == MIQ_F32, MIQ_ERR_UNSUPPORTED, "gptq_gemv: x dtype");
  MIQ_REQUIRE(out_dtype == MIQ_F16 || out_dtype == MIQ_F32, MIQ_ERR_UNSUPPORTED, "gptq_gemv: out dtype");
  hipStream_t st = static_cast<hipStream_t>(stream);
  const int per = 32 / bits;
  // chunk of 64 activations (or 32 when the group is smaller)
  if (gs % 64 == 0 && K % 64 == 0) {
    if (bits == 4) return gemv_mr<4, 64>(x, x_dtype, perm, qweight, qzeros, scales, scales_dtype, bias, out, out_dtype, M, K, N, gs, zero_offset, st);
    return gemv_mr<8, 64>(x, x_dtype, perm, qweight, qzeros, scales, scales_dtype, bias, out, out_dtype, M, K, N, gs, zero_offset, st);
  }
  MIQ_REQUIRE(gs % 32 == 0, MIQ_ERR_UNSUPPORTED, "gptq_gemv: group size %d (needs a multiple of 32)", gs);
  (void)per;
  if (bits == 4) return gemv_mr<4, 32>(x, x_dtype, perm, qweight, qzeros, scales, scales_dtype, bias, out, out_dtype, M, K, N, gs, zero_offset, st);
  return gemv_mr<8, 32>(x, x_dtype, perm, qweight, qzeros, scales, scales_dtype, bias, out, out_dtype, M, K, N, gs, zero_offset, st);
}
