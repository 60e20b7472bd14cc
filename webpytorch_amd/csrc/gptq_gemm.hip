// GPTQ int4/int8 prefill GEMM on the gfx950 matrix cores (v_mfma_f32_16x16x32_f16).
//
// out[M][N] = x[M][K] (fp16, gathered through perm for act-order) @ W + bias, W in the
// AutoGPTQ layout (see gptq_gemv.hip). Dequantization stays exact: each packed word becomes
// the 8 integers q - (z + zoff) in fp16 (exact: |q - z - zoff| <= 256), the matrix cores
// accumulate x * (q - z) in fp32 (fp16 products are exact in fp32), and the fp32 group scale
// is applied to each chunk's partial sums: acc += s[g][n] * sum_{k in chunk} x[k] (q - z).
//
// Mapping. A workgroup is 4 waves side by side along N; a wave owns 64 columns as 4 MFMA
// column blocks, lane (p, kb) = (lane % 16, lane / 16) holding columns ncol + s = n_wave +
// 4 p + s (s = 0..3, one 16-byte load covers all four) and the k-block kb of each 32-wide
// step. The B operand of an MFMA is one packed word per lane (int4: 8 consecutive k of one
// column; int8: two words); its 8 values come out of the unpack in the order c0 c4 c1 c5 c2
// c6 c3 c7 (int8: c0 c2 c1 c3 c4 c6 c5 c7), so the activations are staged in LDS in that same
// order within each 8-wide k block, which leaves every dot product unchanged. A workgroup
// covers BM = 16 * TM rows of x; the K range is cut into chunks of KC (<= 128, inside one
// group) and, for parallelism, into ksplit slices combined deterministically through the
// workspace exactly as the GEMV does (last-arriving workgroup sums the slices in order).
#include <type_traits>

#include "miq_common.h"

namespace miq {

#ifndef MIQ_GEMM_TARGET_WGS
#define MIQ_GEMM_TARGET_WGS 256
#endif

template <int BITS, int TM, int KC, typename ST, typename OT>
__global__ __launch_bounds__(256) void gptq_gemm_kernel(
    const __half* __restrict__ x, const int32_t* __restrict__ perm, const uint32_t* __restrict__ qw,
    const uint32_t* __restrict__ qz, const ST* __restrict__ sc, const float* __restrict__ bias,
    OT* __restrict__ out, float* __restrict__ ws, int* __restrict__ counters, int M, int K, int N, int gs,
    float zoff, int chunks_per_wg, int ksplit) {
  constexpr int PER = 32 / BITS;
  constexpr int BM = 16 * TM;
  constexpr int STEPS = KC / 32;
  constexpr int RB = BITS == 4 ? 1 : 2;  // 16-byte weight loads per lane and step
  __shared__ __align__(16) _Float16 xs[BM * KC];  // activation chunk [BM][KC], pair order
  __shared__ int is_last;

  const int lane = threadIdx.x & 63;
  const int wave = uniform(threadIdx.x >> 6);
  const int p = lane & 15, kb = lane >> 4;
  const int ncol = blockIdx.x * 256 + wave * 64 + 4 * p;
  const bool colok = ncol < N;
  const bool wave_active = blockIdx.x * 256 + wave * 64 < N;
  const int m0 = blockIdx.y * BM;
  const int ks = blockIdx.z;
  const int nchunks = K / KC;
  const int c0 = ks * chunks_per_wg;
  const int c1 = min(nchunks, c0 + chunks_per_wg);
  const int NZ = N / PER;
  const int zshift = (ncol % PER) * BITS;

  float4v acc[TM][4];
#pragma unroll
  for (int t = 0; t < TM; ++t)
#pragma unroll
    for (int s = 0; s < 4; ++s) acc[t][s] = (float4v){0.f, 0.f, 0.f, 0.f};

  for (int c = c0; c < c1; ++c) {
    const int kc0 = c * KC;
    // ---- weights, scales and zeros of the chunk (issued before the activations are staged) ----
    // lanes past N hold zero weights: the matrix cores read every lane's operands, so no lane
    // of a wave may skip the MFMA (their outputs are dropped at the end)
    uint4 bw[STEPS][RB];
#pragma unroll
    for (int st = 0; st < STEPS; ++st)
#pragma unroll
      for (int rb = 0; rb < RB; ++rb) bw[st][rb] = make_uint4(0u, 0u, 0u, 0u);
    uint4 sraw = make_uint4(0u, 0u, 0u, 0u);
    uint32_t zraw = 0;
    if (colok) {
#pragma unroll
      for (int st = 0; st < STEPS; ++st)
#pragma unroll
        for (int rb = 0; rb < RB; ++rb) {
          const int row = (kc0 + st * 32) / PER + kb * RB + rb;
          bw[st][rb] = *reinterpret_cast<const uint4*>(qw + (size_t)row * N + ncol);
        }
      const int g = kc0 / gs;
      sraw = load_scales4<ST>(sc + (size_t)g * N + ncol);
      zraw = qz[(size_t)g * NZ + ncol / PER];
    }
    // ---- stage the activation chunk ----
    __syncthreads();  // the previous chunk's reads are done
    for (int ci = threadIdx.x; ci < BM * KC / 8; ci += 256) {
      const int r = ci / (KC / 8), kk = (ci - r * (KC / 8)) * 8;
      const int k = kc0 + kk;
      float v[8];
      if (m0 + r < M) {
        const __half* xr = x + (size_t)(m0 + r) * K;
        if (perm) {
#pragma unroll
          for (int j = 0; j < 8; ++j) v[j] = __half2float(xr[perm[k + j]]);
        } else {
          load8(xr + k, v);
        }
      } else {
#pragma unroll
        for (int j = 0; j < 8; ++j) v[j] = 0.f;
      }
      *reinterpret_cast<uint4*>(xs + r * KC + kk) = pack8_pairs<BITS>(v);
    }
    __syncthreads();
    if (!wave_active) continue;  // wave-uniform: the whole wave is past N

    // ---- zero points folded into the fp16 conversion: (1024 + q) - (1024 + z + zoff) ----
    half2v zl[4], zh[4];
    zero_pairs<BITS>(zraw >> zshift, zoff, zl, zh);
    float4v part[TM][4];
#pragma unroll
    for (int t = 0; t < TM; ++t)
#pragma unroll
      for (int s = 0; s < 4; ++s) part[t][s] = (float4v){0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int st = 0; st < STEPS; ++st) {
      half8v bf[4];
#pragma unroll
      for (int s = 0; s < 4; ++s) bf[s] = b_fragment<BITS>(bw[st], s, zl[s], zh[s]);
#pragma unroll
      for (int t = 0; t < TM; ++t) {
        const half8v af = *reinterpret_cast<const half8v*>(xs + (16 * t + p) * KC + st * 32 + 8 * kb);
#pragma unroll
        for (int s = 0; s < 4; ++s) part[t][s] = __builtin_amdgcn_mfma_f32_16x16x32_f16(af, bf[s], part[t][s], 0, 0, 0);
      }
    }
    float sf[4];
    scales4<ST>(sraw, sf);
#pragma unroll
    for (int t = 0; t < TM; ++t)
#pragma unroll
      for (int s = 0; s < 4; ++s)
#pragma unroll
        for (int r = 0; r < 4; ++r) acc[t][s][r] = fmaf(sf[s], part[t][s][r], acc[t][s][r]);
  }

  // ---- epilogue: D[row = 16 t + 4 kb + r][col = ncol + s] = acc[t][s][r] ----
  if (ksplit == 1) {
    if (!colok) return;
    float b4[4] = {0.f, 0.f, 0.f, 0.f};
    if (bias)
#pragma unroll
      for (int s = 0; s < 4; ++s) b4[s] = bias[ncol + s];
#pragma unroll
    for (int t = 0; t < TM; ++t)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int row = m0 + 16 * t + 4 * kb + r;
        if (row >= M) continue;
        OT* o = out + (size_t)row * N + ncol;
#pragma unroll
        for (int s = 0; s < 4; ++s) o[s] = from_f32<OT>(acc[t][s][r] + b4[s]);
      }
    return;
  }
  // split K: device-scope stores of the slice, count in, the last workgroup sums the slices
  if (colok) {
#pragma unroll
    for (int t = 0; t < TM; ++t)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int row = m0 + 16 * t + 4 * kb + r;
        if (row >= M) continue;
        float* d = ws + ((size_t)ks * M + row) * N + ncol;
#pragma unroll
        for (int s = 0; s < 4; ++s) __hip_atomic_store(d + s, acc[t][s][r], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      }
  }
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
  int* ctr = counters + (size_t)blockIdx.y * gridDim.x + blockIdx.x;
  if (threadIdx.x == 0)
    is_last = __hip_atomic_fetch_add(ctr, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == ksplit - 1;
  __syncthreads();
  if (!is_last) return;
  if (colok) {
    const size_t stride = (size_t)M * N;
#pragma unroll
    for (int t = 0; t < TM; ++t)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int row = m0 + 16 * t + 4 * kb + r;
        if (row >= M) continue;
        const float* pp = ws + (size_t)row * N + ncol;
        float sum[4] = {0.f, 0.f, 0.f, 0.f};
        for (int k2 = 0; k2 < ksplit; ++k2) {
          float v[4];
#pragma unroll
          for (int s = 0; s < 4; ++s) v[s] = __hip_atomic_load(pp + k2 * stride + s, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
#pragma unroll
          for (int s = 0; s < 4; ++s) sum[s] += v[s];
        }
        OT* o = out + (size_t)row * N + ncol;
#pragma unroll
        for (int s = 0; s < 4; ++s) o[s] = from_f32<OT>(sum[s] + (bias ? bias[ncol + s] : 0.f));
      }
  }
  if (threadIdx.x == 0) __hip_atomic_store(ctr, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);  // re-armed
}

struct GemmPlan {
  int tm, kc, tiles, mtiles, ksplit, chunks_per_wg;
  size_t counter_bytes, ws_bytes;
};

static int gemm_plan(int M, int K, int N, int gs, bool have_ws, GemmPlan* p) {
  int kc = 0;
  if (gs % 128 == 0) kc = 128;
  else if (gs == 64) kc = 64;
  else if (gs == 32) kc = 32;
  MIQ_REQUIRE(kc, MIQ_ERR_UNSUPPORTED, "gptq_gemm: group size %d (32, 64 or a multiple of 128)", gs);
  p->kc = kc;
  p->tm = M >= 64 ? 4 : (M >= 32 ? 2 : 1);
  p->tiles = (N + 255) / 256;
  p->mtiles = (M + 16 * p->tm - 1) / (16 * p->tm);
  const int nchunks = K / kc;
  const int base = p->tiles * p->mtiles;
  int ksplit = have_ws && base <= kMaxCounters ? (MIQ_GEMM_TARGET_WGS + base - 1) / base : 1;
  if (ksplit > nchunks) ksplit = nchunks;
  if (ksplit < 1) ksplit = 1;
  p->chunks_per_wg = (nchunks + ksplit - 1) / ksplit;
  p->ksplit = (nchunks + p->chunks_per_wg - 1) / p->chunks_per_wg;
  p->counter_bytes = p->ksplit > 1 ? kCounterBytes : 0;
  p->ws_bytes = p->ksplit > 1 ? p->counter_bytes + (size_t)p->ksplit * M * N * 4 : 0;
  return MIQ_OK;
}

template <int BITS, int TM, int KC, typename ST, typename OT>
static int launch_gemm(const GemmPlan& p, const void* x, const int32_t* perm, const int32_t* qw, const int32_t* qz,
                       const void* sc, const float* bias, void* out, void* ws, int M, int K, int N, int gs,
                       float zoff, hipStream_t st) {
  int* counters = p.ksplit > 1 ? static_cast<int*>(ws) : nullptr;
  float* partials = p.ksplit > 1 ? reinterpret_cast<float*>(static_cast<char*>(ws) + p.counter_bytes) : nullptr;
  dim3 grid(p.tiles, p.mtiles, p.ksplit);
  hipLaunchKernelGGL((gptq_gemm_kernel<BITS, TM, KC, ST, OT>), grid, dim3(256), 0, st,
                     static_cast<const __half*>(x), perm, reinterpret_cast<const uint32_t*>(qw),
                     reinterpret_cast<const uint32_t*>(qz), static_cast<const ST*>(sc), bias, static_cast<OT*>(out),
                     partials, counters, M, K, N, gs, zoff, p.chunks_per_wg, p.ksplit);
  return check_launch("gptq_gemm");
}

template <int BITS, int TM, int KC>
static int gemm_types(const GemmPlan& p, const void* x, const int32_t* perm, const int32_t* qw, const int32_t* qz,
                      const void* sc, int sd, const float* bias, void* out, int od, void* ws, int M, int K, int N,
                      int gs, float zoff, hipStream_t st) {
  if (sd == MIQ_F16) {
    if (od == MIQ_F16) return launch_gemm<BITS, TM, KC, __half, __half>(p, x, perm, qw, qz, sc, bias, out, ws, M, K, N, gs, zoff, st);
    return launch_gemm<BITS, TM, KC, __half, float>(p, x, perm, qw, qz, sc, bias, out, ws, M, K, N, gs, zoff, st);
  }
  if (od == MIQ_F16) return launch_gemm<BITS, TM, KC, float, __half>(p, x, perm, qw, qz, sc, bias, out, ws, M, K, N, gs, zoff, st);
  return launch_gemm<BITS, TM, KC, float, float>(p, x, perm, qw, qz, sc, bias, out, ws, M, K, N, gs, zoff, st);
}

template <int BITS>
static int gemm_dispatch(const GemmPlan& p, const void* x, const int32_t* perm, const int32_t* qw, const int32_t* qz,
                         const void* sc, int sd, const float* bias, void* out, int od, void* ws, int M, int K, int N,
                         int gs, float zoff, hipStream_t st) {
#define MIQ_GEMM_CASE(TM, KC) \
  if (p.tm == TM && p.kc == KC) \
    return gemm_types<BITS, TM, KC>(p, x, perm, qw, qz, sc, sd, bias, out, od, ws, M, K, N, gs, zoff, st)
  MIQ_GEMM_CASE(1, 128); MIQ_GEMM_CASE(2, 128); MIQ_GEMM_CASE(4, 128);
  MIQ_GEMM_CASE(1, 64); MIQ_GEMM_CASE(2, 64); MIQ_GEMM_CASE(4, 64);
  MIQ_GEMM_CASE(1, 32); MIQ_GEMM_CASE(2, 32); MIQ_GEMM_CASE(4, 32);
#undef MIQ_GEMM_CASE
  return fail(MIQ_ERR_UNSUPPORTED, "gptq_gemm: no kernel for tm=%d kc=%d", p.tm, p.kc);
}

int check_gptq_dims(const char* who, int K, int N, int gs, int bits);

}  // namespace miq

using namespace miq;

extern "C" int miq_gptq_gemm_workspace(int M, int K, int N, int gs, int bits, size_t* bytes) {
  MIQ_REQUIRE(bytes, MIQ_ERR_INVALID, "gptq_gemm_workspace: null output");
  *bytes = 0;
  int rc = check_gptq_dims("gptq_gemm_workspace", K, N, gs, bits);
  if (rc) return rc;
  MIQ_REQUIRE(M >= 0, MIQ_ERR_INVALID, "gptq_gemm_workspace: M=%d", M);
  if (M == 0) return MIQ_OK;
  GemmPlan p;
  rc = gemm_plan(M, K, N, gs, true, &p);
  if (rc) return rc;
  *bytes = p.ws_bytes;
  return MIQ_OK;
}

extern "C" int miq_gptq_gemm(const void* x, const int32_t* perm, const int32_t* qweight, const int32_t* qzeros,
                             const void* scales, int scales_dtype, const float* bias, void* out, int out_dtype, int M,
                             int K, int N, int gs, int bits, float zero_offset, void* workspace,
                             size_t workspace_bytes, void* stream) {
  int rc = check_gptq_dims("gptq_gemm", K, N, gs, bits);
  if (rc) return rc;
  MIQ_REQUIRE(M >= 0, MIQ_ERR_INVALID, "gptq_gemm: M=%d", M);
  if (M == 0) return MIQ_OK;
  MIQ_REQUIRE(x && qweight && qzeros && scales && out, MIQ_ERR_INVALID, "gptq_gemm: null pointer");
  MIQ_REQUIRE(N % 4 == 0 && K % 32 == 0 && aligned(qweight, 16) && aligned(x, 16) &&
                  aligned(scales, scales_dtype == MIQ_F16 ? 8 : 16),
              MIQ_ERR_ALIGN, "gptq_gemm: x and qweight must be 16-byte aligned, N %% 4 == 0, K %% 32 == 0");
  MIQ_REQUIRE(scales_dtype == MIQ_F16 || scales_dtype == MIQ_F32, MIQ_ERR_UNSUPPORTED, "gptq_gemm: scales dtype");
  MIQ_REQUIRE(out_dtype == MIQ_F16 || out_dtype == MIQ_F32, MIQ_ERR_UNSUPPORTED, "gptq_gemm: out dtype");
  MIQ_REQUIRE(zero_offset == (float)(int)zero_offset && zero_offset >= 0.f && zero_offset <= 8.f, MIQ_ERR_UNSUPPORTED,
              "gptq_gemm: zero_offset %g (the exact fp16 path takes a small integer)", zero_offset);
  GemmPlan p;
  rc = gemm_plan(M, K, N, gs, workspace != nullptr, &p);
  if (rc) return rc;
  if (p.ksplit > 1) {
    MIQ_REQUIRE(workspace_bytes >= p.ws_bytes && aligned(workspace, 256), MIQ_ERR_INVALID,
                "gptq_gemm: workspace of %zu bytes (256-byte aligned) needed, %zu given", p.ws_bytes, workspace_bytes);
  }
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (bits == 4)
    return gemm_dispatch<4>(p, x, perm, qweight, qzeros, scales, scales_dtype, bias, out, out_dtype, workspace, M, K,
                            N, gs, zero_offset, st);
  return gemm_dispatch<8>(p, x, perm, qweight, qzeros, scales, scales_dtype, bias, out, out_dtype, workspace, M, K, N,
                          gs, zero_offset, st);
}
