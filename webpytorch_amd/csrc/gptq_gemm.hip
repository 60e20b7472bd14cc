// GPTQ int4/int8 prefill GEMM on the gfx950 matrix cores (v_mfma_f32_16x16x32_f16).
//
// out[M][N] = x[M][K] (fp16) @ W + bias, W in the AutoGPTQ layout (see gptq_gemv.hip).
// Dequantization stays exact: each packed word becomes the 8 integers q - (z + zoff) in fp16
// (exact: |q - z - zoff| <= 263), the matrix cores accumulate x * (q - z) in fp32 (fp16
// products are exact in fp32), and the fp32 group scale multiplies each stage's partial sums:
// acc += s[g][n] * sum_{k in stage} x[k] (q - z).
//
// Activations. A first pass copies x into the workspace (gathered through perm for act-order)
// with each 8-wide k block reordered the way the code unpack produces the weights: int4
// c0 c4 c1 c5 c2 c6 c3 c7, int8 c0 c2 c1 c3 c4 c6 c5 c7. Every dot product is unchanged, the
// MFMA A operand is then a plain 16-byte read, and the B operand needs no byte shuffling.
//
// Mapping. A workgroup is 4 waves side by side along N; a wave owns 16 TM rows x 16 CB columns
// as TM x CB MFMA tiles (BM = 16 TM, BN = 64 CB). Lane (p, kb) = (lane % 16, lane / 16) holds
// columns ncol + s = n_wave + CB p + s (s < CB; one LDS read gives the CB packed words of a k
// row) and the 8-wide k block kb of each 32-wide MFMA step. Each wave dequantizes its own
// columns, so the unpack is spread over the 16 TM rows it feeds.
//
// Pipeline. K is walked in stages of KC (<= 128, inside one group). A stage's activation rows,
// packed weight rows, scales and zero points are copied global -> LDS by the DMA path of the
// vector memory unit (global_load_lds), so no register holds data on its way to LDS. The
// workgroup's multiplying waves are two halves of 4 (one wave of each half per SIMD, on the same
// columns): stages go in pairs, and half h multiplies stage 2j + h of pair j into accumulators of
// its own. Wave tiles of up to 4 MFMA tiles get 4 more waves that only issue the copies, P2
// pairs ahead (a copy instruction that finds the memory pipeline full stalls the wave that
// issues it; kept on their own waves, those stalls never hold back an MFMA); with larger tiles
// each multiplying wave copies its own stages (measured faster there: three waves per SIMD cap
// the registers at 168, and the copies are then the bound either way). One barrier per pair both publishes the pair that landed and frees the buffers that
// the next copies overwrite; while one multiplying wave of a SIMD waits on LDS, the other keeps
// the matrix core busy. The halves' sums are added at the end (half 0 + half 1, a fixed order). Activation rows sit in LDS with their 16-byte chunks
// XOR-swizzled by row (chunk c of row r at slot c ^ (r mod chunks-per-row)), so the 16 rows that
// one operand read touches fall in different banks.
//
// K may also be split over workgroups (ksplit) when the tile grid alone is too small for the
// chip; slices are combined deterministically through the workspace, the last workgroup to
// arrive summing them in slice order, as the GEMV does.
//
// Placement. Workgroups are dispatched round-robin over the 8 XCDs, each with its own L2; the
// tile order is remapped so that the workgroups on one XCD share weight columns (same column
// tile and K slice, different row tiles).
#include <algorithm>
#include <type_traits>

#include "miq_common.h"

namespace miq {

constexpr int kGemmTargetWgs = 256;  // a tile grid of this many workgroups needs no K split


constexpr int kXCDs = 8;
constexpr int kLdsBytes = 160 * 1024;

// 16 bytes stored with device scope (sc1: written through the XCD's L2, so that workgroups on
// other XCDs read it). Not counted by the compiler's wait counters: the caller waits with
// s_waitcnt before publishing.
__device__ __forceinline__ void store_agent16(float* p, float4v v) {
  asm volatile("global_store_dwordx4 %0, %1, off sc1" ::"v"(p), "v"(v) : "memory");
}
__device__ __forceinline__ uint64_t pack_f2(float a, float b) {
  return (uint64_t)__float_as_uint(a) | ((uint64_t)__float_as_uint(b) << 32);
}

// 8 fp16 in k order (16 bytes: words (h0,h1) (h2,h3) (h4,h5) (h6,h7)) into the unpack's order
template <int BITS> __device__ __forceinline__ uint4 pair_order8(uint4 v) {
  if constexpr (BITS == 4)  // (h0,h4) (h1,h5) (h2,h6) (h3,h7)
    return make_uint4((v.x & 0xFFFFu) | (v.z << 16), (v.x >> 16) | (v.z & 0xFFFF0000u),
                      (v.y & 0xFFFFu) | (v.w << 16), (v.y >> 16) | (v.w & 0xFFFF0000u));
  else  // (h0,h2) (h1,h3) (h4,h6) (h5,h7)
    return make_uint4((v.x & 0xFFFFu) | (v.y << 16), (v.x >> 16) | (v.y & 0xFFFF0000u),
                      (v.z & 0xFFFFu) | (v.w << 16), (v.z >> 16) | (v.w & 0xFFFF0000u));
}

// xp = x with each 8-wide k block in pair order, stored stage-major: xp[k / KC][m][k % KC]. A
// stage of a row tile is then one contiguous block, which spreads its reads over all L2
// channels (rows of x are 2 K bytes apart, a power of two for the usual K, and would all land
// in the same few channels).
//
// One workgroup per row of x; every thread issues four 16-byte loads before it stores anything.
// With perm (act-order columns), the row goes to LDS first (coalesced) and each output chunk
// gathers its 8 values from there through its 8 permutation indices, which are loaded before
// the row. Grid (M), dynamic LDS 2 K bytes with perm.
template <int BITS, bool PERM>
__global__ __launch_bounds__(256) void stage_rows_kernel(const __half* __restrict__ x, const int32_t* __restrict__ perm,
                                                         __half* __restrict__ xp, int M, int K, int KC) {
  extern __shared__ __align__(16) unsigned short srow[];  // [K] (perm only)
  constexpr int U = 4;
  const int m = blockIdx.x, nch = K / 8;
  const uint4* src = reinterpret_cast<const uint4*>(x + (size_t)m * K);
  auto dst = [&](int i) {
    const int k = i * 8;
    return reinterpret_cast<uint4*>(xp + ((size_t)(k / KC) * M + m) * KC + k % KC);
  };
  if constexpr (PERM) {
    // rows up to 256 U chunks (K <= 8192) keep their permutation indices in registers across
    // the barrier; longer rows reload them per pass
    const int4* p4 = reinterpret_cast<const int4*>(perm);
    int4 pa[U], pb[U];
    auto load_perm = [&](int q0) {
#pragma unroll
      for (int j = 0; j < U; ++j) {
        const int i = min(q0 + 256 * j, nch - 1);
        pa[j] = p4[2 * i];
        pb[j] = p4[2 * i + 1];
      }
    };
    load_perm(threadIdx.x);
    for (int q0 = threadIdx.x; q0 < nch; q0 += 256 * U) {
      uint4 v[U];
#pragma unroll
      for (int j = 0; j < U; ++j) v[j] = src[min(q0 + 256 * j, nch - 1)];
#pragma unroll
      for (int j = 0; j < U; ++j)
        if (q0 + 256 * j < nch) reinterpret_cast<uint4*>(srow)[q0 + 256 * j] = v[j];
    }
    __syncthreads();
    for (int q0 = threadIdx.x; q0 < nch; q0 += 256 * U) {
      if (q0 != (int)threadIdx.x) load_perm(q0);
#pragma unroll
      for (int j = 0; j < U; ++j) {
        if (q0 + 256 * j >= nch) break;
        const uint4 v = make_uint4(srow[(unsigned)pa[j].x] | ((uint32_t)srow[(unsigned)pa[j].y] << 16),
                                   srow[(unsigned)pa[j].z] | ((uint32_t)srow[(unsigned)pa[j].w] << 16),
                                   srow[(unsigned)pb[j].x] | ((uint32_t)srow[(unsigned)pb[j].y] << 16),
                                   srow[(unsigned)pb[j].z] | ((uint32_t)srow[(unsigned)pb[j].w] << 16));
        *dst(q0 + 256 * j) = pair_order8<BITS>(v);
      }
    }
  } else {
    for (int q0 = threadIdx.x; q0 < nch; q0 += 256 * U) {
      uint4 v[U];
#pragma unroll
      for (int j = 0; j < U; ++j) v[j] = src[min(q0 + 256 * j, nch - 1)];
#pragma unroll
      for (int j = 0; j < U; ++j)
        if (q0 + 256 * j < nch) *dst(q0 + 256 * j) = pair_order8<BITS>(v[j]);
    }
  }
}

// fp32 activations through the fp16 matrix cores: row m of x is scaled by 2^s (s making its
// largest |x| just below 2^15) and split into hi = fp16(x 2^s) and lo = fp16(x 2^s - hi), staged
// as rows m and M + m of a 2M-row problem (about 22 significant bits relative to the row's
// largest value, no fp16 range limit; NaN or infinite rows keep scale 1 and propagate). The
// GEMM's two result rows are added and scaled back by 2^-s (exact).
__device__ __forceinline__ int f32_row_exp(float m) {
  if (!(m > 0.f) || !(m <= 3.4e38f)) return 0;
  int ex;
  frexpf(m, &ex);
  return min(max(15 - ex, -126), 126);  // any finite maximum lands below 2^15; 2^s stays finite
}

// Stage row m of fp32 x (gathered through perm if PERM) as hi (row m) and lo (row M + m) of the
// 2M-row stage-major pair-ordered layout, and record the row's largest |x| (NaN if it holds one)
// in rmax[m] for the combine. The row goes through LDS (its maximum sets the scale before any
// value is split). Grid (M), dynamic LDS 4 K bytes.
template <int BITS, bool PERM>
__global__ __launch_bounds__(256) void stage_rows_f32_kernel(const float* __restrict__ x, const int32_t* __restrict__ perm,
                                                             float* __restrict__ rmax, __half* __restrict__ xp, int M,
                                                             int K, int KC) {
  extern __shared__ __align__(16) float frow[];  // [K]
  __shared__ float wmax[4];
  __shared__ int wnan[4];
  const int m = blockIdx.x, nch = K / 8, M2 = 2 * M, lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
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
  const float sc = ldexpf(1.f, f32_row_exp(mx));
  for (int i = threadIdx.x; i < nch; i += 256) {
    float v[8];
    if constexpr (PERM) {
      const int4 pa = reinterpret_cast<const int4*>(perm)[2 * i], pb = reinterpret_cast<const int4*>(perm)[2 * i + 1];
      const int idx[8] = {pa.x, pa.y, pa.z, pa.w, pb.x, pb.y, pb.z, pb.w};
#pragma unroll
      for (int j = 0; j < 8; ++j) v[j] = frow[(unsigned)idx[j]];
    } else {
#pragma unroll
      for (int j = 0; j < 8; ++j) v[j] = frow[8 * i + j];
    }
    uint32_t hi[4], lo[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const float a0 = v[2 * j] * sc, a1 = v[2 * j + 1] * sc;
      const __half h0 = __float2half_rn(a0), h1 = __float2half_rn(a1);
      hi[j] = (uint32_t)__half_as_ushort(h0) | ((uint32_t)__half_as_ushort(h1) << 16);
      lo[j] = (uint32_t)__half_as_ushort(__float2half_rn(a0 - __half2float(h0))) |
              ((uint32_t)__half_as_ushort(__float2half_rn(a1 - __half2float(h1))) << 16);
    }
    const int k = i * 8;
    *reinterpret_cast<uint4*>(xp + ((size_t)(k / KC) * M2 + m) * KC + k % KC) =
        pair_order8<BITS>(make_uint4(hi[0], hi[1], hi[2], hi[3]));
    *reinterpret_cast<uint4*>(xp + ((size_t)(k / KC) * M2 + M + m) * KC + k % KC) =
        pair_order8<BITS>(make_uint4(lo[0], lo[1], lo[2], lo[3]));
  }
}

// out[m][n] = (y2[m][n] + y2[M + m][n]) 2^-s(m) + bias[n]. Grid (N/4/256 rounded up, M).
template <typename OT>
__global__ __launch_bounds__(256) void combine_rows_kernel(const float* __restrict__ y2, const float* __restrict__ rmax,
                                                           const float* __restrict__ bias, OT* __restrict__ out, int M,
                                                           int N) {
  const int m = blockIdx.y, n = (blockIdx.x * 256 + threadIdx.x) * 4;
  if (n >= N) return;
  const float un = ldexpf(1.f, -f32_row_exp(rmax[m]));
  const float4 a = *reinterpret_cast<const float4*>(y2 + (size_t)m * N + n);
  const float4 b = *reinterpret_cast<const float4*>(y2 + (size_t)(M + m) * N + n);
  const float r[4] = {(a.x + b.x) * un, (a.y + b.y) * un, (a.z + b.z) * un, (a.w + b.w) * un};
#pragma unroll
  for (int j = 0; j < 4; ++j) out[(size_t)m * N + n + j] = from_f32<OT>(bias ? r[j] + bias[n + j] : r[j]);
}

// Launches the staging of x (gathered through perm if non-null) into xp with stage width KC.
template <int BITS>
static int stage_rows(const __half* x, const int32_t* perm, __half* xp, int M, int K, int KC, hipStream_t st) {
  if (perm) {
    const size_t lds = (size_t)K * 2;
    if (lds > 64 * 1024) {
      const int rc = require_lds("gptq_gemm gather", lds);
      if (rc) return rc;
    }
    hipLaunchKernelGGL((stage_rows_kernel<BITS, true>), dim3(M), dim3(256), lds, st, x, perm, xp, M, K, KC);
  } else {
    hipLaunchKernelGGL((stage_rows_kernel<BITS, false>), dim3(M), dim3(256), 0, st, x, perm, xp, M, K, KC);
  }
  return check_launch("gptq_gemm staging");
}

template <int BITS, int TM, int CB, int KC, typename ST> struct GemmShape {
  static constexpr int PER = 32 / BITS;
  static constexpr int BM = 16 * TM, BN = 64 * CB;
  static constexpr int STEPS = KC / 32;
  static constexpr int RB = BITS == 4 ? 1 : 2;    // packed rows per lane and MFMA step
  static constexpr int AROW = KC * 2;             // bytes of one activation row of a stage
  static constexpr int CPR = AROW / 16;           // 16-byte chunks per row
  static constexpr int RPI = 1024 / AROW;         // rows per activation DMA (64 lanes x 16 B)
  static constexpr int NA = BM / RPI;             // activation DMAs per stage
  static constexpr int BROWS = KC / PER;          // packed weight rows per stage
  static constexpr int BROWB = BN * 4;            // bytes per packed row of the tile
  static constexpr int NB = BROWS * BROWB / 1024; // weight DMAs per stage (16-byte lanes)
  static constexpr int SB = BN * (int)sizeof(ST); // scale bytes per stage
  static constexpr int NS = SB / 256;             // scale DMAs (4-byte lanes)
  static constexpr int NI = NA + NB + NS + 1;     // + one zero-point DMA
  static constexpr int NIW = (NI + 3) / 4;        // per wave (the last ones repeat the zero DMA)
  static constexpr int A_OFF = 0, B_OFF = BM * AROW, S_OFF = B_OFF + BROWS * BROWB, Z_OFF = S_OFF + SB;
  static constexpr int STAGE = Z_OFF + 256;
  static constexpr int NB2 = 6 * STAGE + 64 <= kLdsBytes ? 3 : 2;  // buffered stage pairs
  static constexpr int NBUF = 2 * NB2;
  static constexpr int P2 = NB2 - 1;              // pairs in flight ahead of the one multiplied
  static constexpr int RED = 4 * TM * CB * 4 * 64 * 4;  // one half's accumulators, for the final sum
  static_assert(BM % RPI == 0 && (BROWS * BROWB) % 1024 == 0 && SB % 256 == 0, "whole DMAs");
  static_assert(BN / PER <= 64, "zero points of a tile fit one DMA");
  static constexpr int LDS = NBUF * STAGE > RED ? NBUF * STAGE : RED;
  static constexpr bool COPIERS = TM * CB <= 4;   // 4 waves that only copy
  static constexpr int THREADS = COPIERS ? 768 : 512;
  static_assert(4 * STAGE + 64 <= kLdsBytes && LDS + 64 <= kLdsBytes, "LDS");
  static_assert(4 * NIW < 64, "vmcnt range");
};

// Waves w and w + 4 own the same columns and take alternate stages; wave w + 8, if any, copies.
template <int BITS, int TM, int CB, int KC, typename ST, typename OT>
__global__ __attribute__((amdgpu_flat_work_group_size(1, TM * CB <= 4 ? 768 : 512),
                          amdgpu_waves_per_eu(TM * CB <= 4 ? 3 : 2, TM * CB <= 4 ? 3 : 2))) void gptq_gemm_kernel(
    const __half* __restrict__ xp, const uint32_t* __restrict__ qw, const uint32_t* __restrict__ qz,
    const ST* __restrict__ sc, const float* __restrict__ bias, OT* __restrict__ out, float* __restrict__ ws,
    int* __restrict__ counters, int M, int K, int N, int gs, float zoff, int stages_per_wg, int ksplit, int ntiles,
    int mtiles) {
  using G = GemmShape<BITS, TM, CB, KC, ST>;
  constexpr int PER = G::PER, STEPS = G::STEPS, RB = G::RB, NBUF = G::NBUF, NB2 = G::NB2, P2 = G::P2, NIW = G::NIW;
  __shared__ __align__(16) char lds[G::LDS];
  __shared__ int is_last;

  // ---- tile of this workgroup: XCD-major order, row tiles fastest ----
  const int T = (int)gridDim.x, L = (int)blockIdx.x;
  const int Lp = T % kXCDs == 0 ? (L % kXCDs) * (T / kXCDs) + L / kXCDs : L;
  const int mtile = Lp % mtiles;
  const int rest = Lp / mtiles;
  const int ks = rest % ksplit;
  const int ntile = rest / ksplit;

  const int tid = threadIdx.x, lane = tid & 63;
  const bool copier = G::COPIERS && uniform(tid >> 6) >= 8;  // waves 8..11 issue the copies
  const int half = (uniform(tid >> 6) >> 2) & 1;  // which stage of each pair this wave multiplies
  const int wave = uniform(tid >> 6) & 3;  // column group / copy slot (the range lets each copy's kind fold)
  const int p = lane & 15, kb = lane >> 4;
  const int n0 = ntile * G::BN;
  const int cl = wave * 16 * CB + CB * p;  // the lane's first column within the tile
  const int ncol = n0 + cl;
  const bool colok = ncol < N;
  const int m0 = mtile * G::BM;
  const int nst = K / KC;
  const int st0 = ks * stages_per_wg;
  const int st1 = min(nst, st0 + stages_per_wg);
  const int last = st1 - 1;
  const int NZ = N / PER;
  const uint32_t lds0 = lds_addr(lds);

  // ---- copy j of one stage into LDS buffer buf: instruction i = wave + 4 j of the stage.
  // Rows past M and columns past N re-read the last valid row / column (in bounds; they only
  // feed outputs that are never stored).
  auto issue_one = [&](int s, int buf, int j) __attribute__((always_inline)) {
    const uint32_t base = lds0 + buf * G::STAGE;
    const int g = s * KC / gs;
    const int i = wave + 4 * j;  // wave-uniform
    if (i < G::NA) {
      const int rloc = i * G::RPI + lane / G::CPR, slot = lane % G::CPR;
      const int chunk = slot ^ (rloc % G::CPR);
      const int row = min(m0 + rloc, M - 1);
      dma16(xp + ((size_t)s * M + row) * KC + chunk * 8, uniform(base + G::A_OFF + i * 1024));
    } else if (i < G::NA + G::NB) {
      const int b = i - G::NA;
      const int r = b * (1024 / G::BROWB) + lane / (G::BROWB / 16), c4 = lane % (G::BROWB / 16);
      dma16(qw + (size_t)(s * G::BROWS + r) * N + min(n0 + 4 * c4, N - 4), uniform(base + G::B_OFF + b * 1024));
    } else if (i < G::NA + G::NB + G::NS) {
      const int h = i - G::NA - G::NB;
      constexpr int E = 4 / (int)sizeof(ST);  // scales per lane
      dma4(sc + (size_t)g * N + min(n0 + 64 * E * h + E * lane, N - E), uniform(base + G::S_OFF + 256 * h));
    } else {
      dma4(qz + (size_t)g * NZ + min(n0 / PER + lane, NZ - 1), uniform(base + G::Z_OFF));
    }
  };
  auto issue = [&](int s, int buf) __attribute__((always_inline)) {
#pragma unroll
    for (int j = 0; j < NIW; ++j) issue_one(s, buf, j);
  };

  float4v acc[TM][CB];
#pragma unroll
  for (int t = 0; t < TM; ++t)
#pragma unroll
    for (int s = 0; s < CB; ++s) acc[t][s] = (float4v){0.f, 0.f, 0.f, 0.f};

  // One stage of matrix work. Every LDS read of the stage is issued first, then the weights
  // are unpacked step by step while the MFMAs run.
  auto compute = [&](int buf) __attribute__((always_inline)) {
    const char* stg = lds + buf * G::STAGE;
    uint4 bw[STEPS][RB];
    half8v af[STEPS][TM];
#pragma unroll
    for (int st = 0; st < STEPS; ++st)
#pragma unroll
      for (int rb = 0; rb < RB; ++rb) {
        const char* src = stg + G::B_OFF + ((st * 32) / PER + kb * RB + rb) * G::BROWB + cl * 4;
        if constexpr (CB == 4) {
          bw[st][rb] = *reinterpret_cast<const uint4*>(src);
        } else {
          const uint2 t2 = *reinterpret_cast<const uint2*>(src);
          bw[st][rb] = make_uint4(t2.x, t2.y, 0u, 0u);
        }
      }
    const uint32_t zw = *reinterpret_cast<const uint32_t*>(stg + G::Z_OFF + (cl / PER) * 4) >> ((cl % PER) * BITS);
#pragma unroll
    for (int st = 0; st < STEPS; ++st)
#pragma unroll
      for (int t = 0; t < TM; ++t) {
        const int r = 16 * t + p, chunk = st * 4 + kb;
        af[st][t] = *reinterpret_cast<const half8v*>(stg + G::A_OFF + r * G::AROW + ((chunk ^ (r % G::CPR)) * 16));
      }
    float sf[4];
    if constexpr (CB == 4) {
      scales4<ST>(load_scales4<ST>(reinterpret_cast<const ST*>(stg + G::S_OFF) + cl), sf);
    } else {
      const ST* sp = reinterpret_cast<const ST*>(stg + G::S_OFF) + cl;
      sf[0] = to_f32(sp[0]);
      sf[1] = to_f32(sp[1]);
    }
    __builtin_amdgcn_sched_barrier(0);
    half2v zl[4], zh[4];
    zero_pairs<BITS>(zw, zoff, zl, zh);
    float4v part[TM][CB];
#pragma unroll
    for (int t = 0; t < TM; ++t)
#pragma unroll
      for (int s = 0; s < CB; ++s) part[t][s] = (float4v){0.f, 0.f, 0.f, 0.f};
    // the unpack runs one step ahead of the MFMAs, and the scheduling pattern below puts a few
    // unpack instructions behind each MFMA: the SIMD issues them while the matrix core works
    half8v bf[CB], bn[CB];
#pragma unroll
    for (int s = 0; s < CB; ++s) bn[s] = b_fragment<BITS>(bw[0], s, zl[s], zh[s]);
#pragma unroll
    for (int st = 0; st < STEPS; ++st) {
#pragma unroll
      for (int s = 0; s < CB; ++s) bf[s] = bn[s];
      if (st + 1 < STEPS) {
#pragma unroll
        for (int s = 0; s < CB; ++s) bn[s] = b_fragment<BITS>(bw[st + 1], s, zl[s], zh[s]);
      }
#pragma unroll
      for (int t = 0; t < TM; ++t)
#pragma unroll
        for (int s = 0; s < CB; ++s)
          part[t][s] = __builtin_amdgcn_mfma_f32_16x16x32_f16(af[st][t], bf[s], part[t][s], 0, 0, 0);
    }
#pragma unroll
    for (int t = 0; t < TM; ++t)
#pragma unroll
      for (int s = 0; s < CB; ++s)
#pragma unroll
        for (int r = 0; r < 4; ++r) acc[t][s][r] = fmaf(sf[s], part[t][s][r], acc[t][s][r]);
  };

  // ---- pipeline: pairs of stages, half h owning stage st0 + 2 j + h of pair j (buffer
  // 2 (j mod NB2) + h); the copying waves run P2 pairs ahead ----
  const int nst_wg = st1 - st0;
  const int nmine = (nst_wg - half + 1) / 2;  // stages of this half (pairs 0 .. nmine - 1)
  const int npairs = (nst_wg + 1) / 2;
  auto issue_pair = [&](int q) __attribute__((always_inline)) {
    const int b = 2 * (q % NB2);
    issue(st0 + 2 * q, b);
    if (2 * q + 1 < nst_wg) issue(st0 + 2 * q + 1, b + 1);
  };
  if constexpr (G::COPIERS) {
    if (copier) {
#pragma unroll
      for (int q = 0; q < P2; ++q)
        if (q < npairs) issue_pair(q);
    }
    for (int j = 0; j < npairs; ++j) {
      // a copying wave's copies of pair j are done once only those of its later pairs (at most
      // P2 - 1 <= 1, issued after them) remain; the barrier makes every copy of pair j visible
      // and tells the copying waves that pair j - 1, whose buffers the next copies reuse, has
      // been multiplied
      if (copier) {
        const int nxt = j + 1 < npairs && P2 >= 2 ? (2 * (j + 1) + 1 < nst_wg ? 2 : 1) : 0;  // stages of pair j + 1
        if (nxt == 2) wait_vmcnt<2 * NIW>();
        else if (nxt == 1) wait_vmcnt<NIW>();
        else wait_vmcnt<0>();
      }
      __syncthreads();
      if (copier) {
        if (j + P2 < npairs) issue_pair(j + P2);
      } else if (j < nmine) {
        compute(2 * (j % NB2) + half);
      }
    }
  } else {
#pragma unroll
    for (int q = 0; q < P2; ++q)
      if (q < nmine) issue(st0 + 2 * q + half, 2 * q + half);
    for (int j = 0; j < npairs; ++j) {
      // this wave's copies of pair j are done once only those of its later pairs (at most
      // P2 - 1 <= 1, issued after them) remain
      const int later = min(P2 - 1, max(0, nmine - 1 - j));
      if (P2 >= 2 && later >= 1) wait_vmcnt<NIW>();
      else wait_vmcnt<0>();
      __syncthreads();
      if (j + P2 < nmine) issue(st0 + 2 * (j + P2) + half, 2 * ((j + P2) % NB2) + half);
      if (j < nmine) compute(2 * (j % NB2) + half);
    }
  }

  // ---- the two halves' sums: half 1 through LDS (the stage buffers are free once every wave
  // has passed the barrier), half 0 adds them ----
  __syncthreads();
  {
    float* red = reinterpret_cast<float*>(lds) + (size_t)wave * (TM * CB * 4 * 64) + lane;
    if (half == 1 && !copier) {
#pragma unroll
      for (int t = 0; t < TM; ++t)
#pragma unroll
        for (int s = 0; s < CB; ++s)
#pragma unroll
          for (int r = 0; r < 4; ++r) red[((t * CB + s) * 4 + r) * 64] = acc[t][s][r];
    }
    __syncthreads();
    if (half == 0 && !copier) {
#pragma unroll
      for (int t = 0; t < TM; ++t)
#pragma unroll
        for (int s = 0; s < CB; ++s)
#pragma unroll
          for (int r = 0; r < 4; ++r) acc[t][s][r] += red[((t * CB + s) * 4 + r) * 64];
    }
  }
  const bool producer = copier || half == 1;  // from here on, only the barriers

  // ---- epilogue: D[row = m0 + 16 t + 4 kb + r][col = ncol + s] = acc[t][s][r] ----
  if (ksplit == 1) {
    if (producer || !colok) return;
    float bv[CB];
#pragma unroll
    for (int s = 0; s < CB; ++s) bv[s] = bias ? bias[ncol + s] : 0.f;
#pragma unroll
    for (int t = 0; t < TM; ++t)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int row = m0 + 16 * t + 4 * kb + r;
        if (row >= M) continue;
        OT* o = out + (size_t)row * N + ncol;
#pragma unroll
        for (int s = 0; s < CB; ++s) o[s] = from_f32<OT>(acc[t][s][r] + bv[s]);
      }
    return;
  }
  // split K: device-scope stores of the slice, count in, the last workgroup sums the slices
  // (the producer waves take part in the barriers only)
  if (!producer && colok) {
#pragma unroll
    for (int t = 0; t < TM; ++t)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int row = m0 + 16 * t + 4 * kb + r;
        if (row >= M) continue;
        float* d = ws + ((size_t)ks * M + row) * N + ncol;
        if constexpr (CB == 4) {
          store_agent16(d, (float4v){acc[t][0][r], acc[t][1][r], acc[t][2][r], acc[t][3][r]});
        } else {
          __hip_atomic_store(reinterpret_cast<uint64_t*>(d), pack_f2(acc[t][0][r], acc[t][1][r]), __ATOMIC_RELAXED,
                             __HIP_MEMORY_SCOPE_AGENT);
        }
      }
  }
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
  int* ctr = counters + (size_t)ntile * mtiles + mtile;
  if (tid == 0) is_last = __hip_atomic_fetch_add(ctr, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == ksplit - 1;
  __syncthreads();
  if (!is_last || producer) return;
  // the slices are summed in slice order (this workgroup's own slice is still in acc); KU slices
  // per trip keep up to 64 loads in flight per lane. Rows past M and columns past N read row
  // M - 1 / column N - CB (in bounds) and are not stored.
  {
    constexpr int KU = 16 / (TM * CB) > 0 ? 16 / (TM * CB) : 1;
    const int ccol = min(ncol, N - CB);
    float4v sum[TM][CB];
#pragma unroll
    for (int t = 0; t < TM; ++t)
#pragma unroll
      for (int s = 0; s < CB; ++s) sum[t][s] = (float4v){0.f, 0.f, 0.f, 0.f};
    for (int k0 = 0; k0 < ksplit; k0 += KU) {
      float v[KU][TM][4][CB];
#pragma unroll
      for (int u = 0; u < KU; ++u) {
        const int kk = min(k0 + u, ksplit - 1);
#pragma unroll
        for (int t = 0; t < TM; ++t)
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            const uint64_t* pp =
                reinterpret_cast<const uint64_t*>(ws + ((size_t)kk * M + min(m0 + 16 * t + 4 * kb + r, M - 1)) * N + ccol);
#pragma unroll
            for (int s = 0; s < CB; s += 2) {
              const uint64_t w = __hip_atomic_load(pp + s / 2, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
              v[u][t][r][s] = __uint_as_float((uint32_t)w);
              v[u][t][r][s + 1] = __uint_as_float((uint32_t)(w >> 32));
            }
          }
      }
#pragma unroll
      for (int u = 0; u < KU; ++u) {
        if (k0 + u >= ksplit) break;
        const bool own = k0 + u == ks;
#pragma unroll
        for (int t = 0; t < TM; ++t)
#pragma unroll
          for (int s = 0; s < CB; ++s)
#pragma unroll
            for (int r = 0; r < 4; ++r) sum[t][s][r] += own ? acc[t][s][r] : v[u][t][r][s];
      }
    }
    if (colok) {
#pragma unroll
      for (int t = 0; t < TM; ++t)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int row = m0 + 16 * t + 4 * kb + r;
          if (row >= M) continue;
          OT* o = out + (size_t)row * N + ncol;
#pragma unroll
          for (int s = 0; s < CB; ++s) o[s] = from_f32<OT>(sum[t][s][r] + (bias ? bias[ncol + s] : 0.f));
        }
    }
  }
  if (tid == 0) __hip_atomic_store(ctr, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);  // re-armed
}

// wave tiles (TM x CB MFMA tiles per wave) the planner chooses from, largest first
struct WaveTile {
  int tm, cb;
};
constexpr WaveTile kWaveTiles[] = {{4, 4}, {4, 2}, {2, 4}, {2, 2}, {1, 4}, {1, 2}};
constexpr int kNumWaveTiles = 6;

struct GemmPlan {
  int tm, cb, kc, ntiles, mtiles, ksplit, stages_per_wg;
  size_t partial_bytes, xp_bytes, ws_bytes;
};

static int gemm_plan(int M, int K, int N, int gs, int bits, GemmPlan* p) {
  int kc = 0;
  if (gs % 128 == 0) kc = 128;
  else if (gs % 64 == 0) kc = 64;
  else if (gs % 32 == 0) kc = 32;
  MIQ_REQUIRE(kc, MIQ_ERR_UNSUPPORTED, "gptq_gemm: group size %d (a multiple of 32)", gs);
  p->kc = kc;
  // the largest wave tile whose grid covers the chip (no K split); failing that, the one with
  // the most tiles, with K split to make up the rest
  int pick = -1;
  long most = 0;
  int pick_most = 0;
  for (int i = 0; i < kNumWaveTiles; ++i) {
    const long tiles = (long)((M + 16 * kWaveTiles[i].tm - 1) / (16 * kWaveTiles[i].tm)) *
                       ((N + 64 * kWaveTiles[i].cb - 1) / (64 * kWaveTiles[i].cb));
    if (tiles >= kGemmTargetWgs && pick < 0) pick = i;
    if (tiles > most) {
      most = tiles;
      pick_most = i;
    }
  }
  if (pick < 0) pick = pick_most;  // no tile fills the chip alone: the most tiles, K split for the rest
  p->tm = kWaveTiles[pick].tm;
  p->cb = kWaveTiles[pick].cb;
  if (bits == 8 && p->cb == 4 && p->kc == 128) p->kc = 64;  // two stage pairs of LDS
  p->ntiles = (N + 64 * p->cb - 1) / (64 * p->cb);
  p->mtiles = (M + 16 * p->tm - 1) / (16 * p->tm);
  const int nst = K / p->kc;
  const int base = p->ntiles * p->mtiles;
  int ksplit = base <= kMaxCounters ? (kGemmTargetWgs + base - 1) / base : 1;
  if (ksplit > nst) ksplit = nst;
  if (ksplit < 1) ksplit = 1;
  p->stages_per_wg = (nst + ksplit - 1) / ksplit;
  p->ksplit = (nst + p->stages_per_wg - 1) / p->stages_per_wg;
  p->partial_bytes = p->ksplit > 1 ? (size_t)p->ksplit * M * N * 4 : 0;
  p->xp_bytes = ((size_t)M * K * 2 + 255) & ~(size_t)255;
  p->ws_bytes = kCounterBytes + p->partial_bytes + p->xp_bytes;
  return MIQ_OK;
}

template <int BITS, int TM, int CB, int KC, typename ST, typename OT>
static int launch_gemm(const GemmPlan& p, const __half* xp, const int32_t* qw, const int32_t* qz, const void* sc,
                       const float* bias, void* out, void* ws, int M, int K, int N, int gs, float zoff, hipStream_t st) {
  int* counters = static_cast<int*>(ws);
  float* partials = reinterpret_cast<float*>(static_cast<char*>(ws) + kCounterBytes);
  const int grid = p.ntiles * p.mtiles * p.ksplit;
  hipLaunchKernelGGL((gptq_gemm_kernel<BITS, TM, CB, KC, ST, OT>), dim3(grid), dim3(GemmShape<BITS, TM, CB, KC, ST>::THREADS), 0, st, xp,
                     reinterpret_cast<const uint32_t*>(qw), reinterpret_cast<const uint32_t*>(qz),
                     static_cast<const ST*>(sc), bias, static_cast<OT*>(out), partials, counters, M, K, N, gs, zoff,
                     p.stages_per_wg, p.ksplit, p.ntiles, p.mtiles);
  return check_launch("gptq_gemm");
}

template <int BITS, int TM, int CB, int KC>
static int gemm_types(const GemmPlan& p, const __half* xp, const int32_t* qw, const int32_t* qz, const void* sc,
                      int sd, const float* bias, void* out, int od, void* ws, int M, int K, int N, int gs, float zoff,
                      hipStream_t st) {
  if (sd == MIQ_F16) {
    if (od == MIQ_F16)
      return launch_gemm<BITS, TM, CB, KC, __half, __half>(p, xp, qw, qz, sc, bias, out, ws, M, K, N, gs, zoff, st);
    return launch_gemm<BITS, TM, CB, KC, __half, float>(p, xp, qw, qz, sc, bias, out, ws, M, K, N, gs, zoff, st);
  }
  if (od == MIQ_F16)
    return launch_gemm<BITS, TM, CB, KC, float, __half>(p, xp, qw, qz, sc, bias, out, ws, M, K, N, gs, zoff, st);
  return launch_gemm<BITS, TM, CB, KC, float, float>(p, xp, qw, qz, sc, bias, out, ws, M, K, N, gs, zoff, st);
}

template <int BITS, int KC>
static int gemm_tiles(const GemmPlan& p, const __half* xp, const int32_t* qw, const int32_t* qz, const void* sc,
                      int sd, const float* bias, void* out, int od, void* ws, int M, int K, int N, int gs, float zoff,
                      hipStream_t st) {
  if (p.tm == 4 && p.cb == 2) return gemm_types<BITS, 4, 2, KC>(p, xp, qw, qz, sc, sd, bias, out, od, ws, M, K, N, gs, zoff, st);
  if (p.tm == 2 && p.cb == 2) return gemm_types<BITS, 2, 2, KC>(p, xp, qw, qz, sc, sd, bias, out, od, ws, M, K, N, gs, zoff, st);
  if (p.tm == 1 && p.cb == 2) return gemm_types<BITS, 1, 2, KC>(p, xp, qw, qz, sc, sd, bias, out, od, ws, M, K, N, gs, zoff, st);
  if constexpr (BITS == 4 || KC < 128) {  // int8 weights with 4 columns a lane take 64-wide stages
    if (p.tm == 4 && p.cb == 4) return gemm_types<BITS, 4, 4, KC>(p, xp, qw, qz, sc, sd, bias, out, od, ws, M, K, N, gs, zoff, st);
    if (p.tm == 2 && p.cb == 4) return gemm_types<BITS, 2, 4, KC>(p, xp, qw, qz, sc, sd, bias, out, od, ws, M, K, N, gs, zoff, st);
    if (p.tm == 1 && p.cb == 4) return gemm_types<BITS, 1, 4, KC>(p, xp, qw, qz, sc, sd, bias, out, od, ws, M, K, N, gs, zoff, st);
  }
  return ::miq::fail(MIQ_ERR_UNSUPPORTED, "gptq_gemm: no kernel for tile %dx%d, stage %d", p.tm, p.cb, KC);
}

template <int BITS>
static int gemm_dispatch(const GemmPlan& p, const __half* xp, const int32_t* qw, const int32_t* qz, const void* sc,
                         int sd, const float* bias, void* out, int od, void* ws, int M, int K, int N, int gs,
                         float zoff, hipStream_t st) {
  if (p.kc == 128) return gemm_tiles<BITS, 128>(p, xp, qw, qz, sc, sd, bias, out, od, ws, M, K, N, gs, zoff, st);
  if (p.kc == 64) return gemm_tiles<BITS, 64>(p, xp, qw, qz, sc, sd, bias, out, od, ws, M, K, N, gs, zoff, st);
  return gemm_tiles<BITS, 32>(p, xp, qw, qz, sc, sd, bias, out, od, ws, M, K, N, gs, zoff, st);
}

int check_gptq_dims(const char* who, int K, int N, int gs, int bits);

// Workspace layout of the fp32-activation GEMM: the 2M-row GEMM's own workspace (counters,
// partials, staged rows), then its fp32 result [2M][N], then the row maxima [M].
struct F32Plan {
  GemmPlan g;
  size_t y2_off, rmax_off, ws_bytes;
};
static int f32_plan(int M, int K, int N, int gs, int bits, F32Plan* p) {
  int rc = gemm_plan(2 * M, K, N, gs, bits, &p->g);
  if (rc) return rc;
  p->y2_off = (p->g.ws_bytes + 255) & ~(size_t)255;
  p->rmax_off = p->y2_off + (((size_t)2 * M * N * 4 + 255) & ~(size_t)255);
  p->ws_bytes = p->rmax_off + (((size_t)M * 4 + 255) & ~(size_t)255);
  return MIQ_OK;
}

}  // namespace miq

using namespace miq;

extern "C" int miq_gptq_gemm_f32x_workspace(int M, int K, int N, int gs, int bits, size_t* bytes) {
  MIQ_REQUIRE(bytes, MIQ_ERR_INVALID, "gptq_gemm_f32x_workspace: null output");
  *bytes = 0;
  int rc = check_gptq_dims("gptq_gemm_f32x_workspace", K, N, gs, bits);
  if (rc) return rc;
  MIQ_REQUIRE(M >= 0, MIQ_ERR_INVALID, "gptq_gemm_f32x_workspace: M=%d", M);
  if (M == 0) return MIQ_OK;
  F32Plan p;
  rc = f32_plan(M, K, N, gs, bits, &p);
  if (rc) return rc;
  *bytes = p.ws_bytes;
  return MIQ_OK;
}

extern "C" int miq_gptq_gemm_f32x(const float* x, const int32_t* perm, const int32_t* qweight, const int32_t* qzeros,
                                  const void* scales, int scales_dtype, const float* bias, void* out, int out_dtype,
                                  int M, int K, int N, int gs, int bits, float zero_offset, void* workspace,
                                  size_t workspace_bytes, void* stream) {
  int rc = check_gptq_dims("gptq_gemm_f32x", K, N, gs, bits);
  if (rc) return rc;
  MIQ_REQUIRE(M >= 0, MIQ_ERR_INVALID, "gptq_gemm_f32x: M=%d", M);
  if (M == 0) return MIQ_OK;
  MIQ_REQUIRE(x && qweight && qzeros && scales && out, MIQ_ERR_INVALID, "gptq_gemm_f32x: null pointer");
  MIQ_REQUIRE(N % 4 == 0 && K % 32 == 0 && aligned(qweight, 16) && aligned(x, 16) && aligned(scales, 4) &&
                  (!perm || aligned(perm, 16)),
              MIQ_ERR_ALIGN, "gptq_gemm_f32x: x, qweight and perm must be 16-byte aligned, N %% 4 == 0, K %% 32 == 0");
  MIQ_REQUIRE(scales_dtype == MIQ_F16 || scales_dtype == MIQ_F32, MIQ_ERR_UNSUPPORTED, "gptq_gemm_f32x: scales dtype");
  MIQ_REQUIRE(out_dtype == MIQ_F16 || out_dtype == MIQ_F32, MIQ_ERR_UNSUPPORTED, "gptq_gemm_f32x: out dtype");
  MIQ_REQUIRE(zero_offset == (float)(int)zero_offset && zero_offset >= 0.f && zero_offset <= 8.f, MIQ_ERR_UNSUPPORTED,
              "gptq_gemm_f32x: zero_offset %g (the exact fp16 path takes a small integer)", zero_offset);
  MIQ_REQUIRE(K <= 32768, MIQ_ERR_UNSUPPORTED, "gptq_gemm_f32x: K=%d > 32768 (a row is staged in LDS)", K);
  F32Plan p;
  rc = f32_plan(M, K, N, gs, bits, &p);
  if (rc) return rc;
  MIQ_REQUIRE(workspace && workspace_bytes >= p.ws_bytes && aligned(workspace, 256), MIQ_ERR_INVALID,
              "gptq_gemm_f32x: workspace of %zu bytes (256-byte aligned) needed, %zu given", p.ws_bytes, workspace_bytes);
  hipStream_t st = static_cast<hipStream_t>(stream);
  char* ws = static_cast<char*>(workspace);
  __half* xp = reinterpret_cast<__half*>(ws + kCounterBytes + p.g.partial_bytes);
  float* y2 = reinterpret_cast<float*>(ws + p.y2_off);
  float* rmax = reinterpret_cast<float*>(ws + p.rmax_off);
  const size_t lds = (size_t)K * 4;
  if (lds > 64 * 1024 && (rc = require_lds("gptq_gemm_f32x staging", lds))) return rc;
#define MIQ_F32_STAGE(B, P)                                                                                      \
  hipLaunchKernelGGL((stage_rows_f32_kernel<B, P>), dim3(M), dim3(256), lds, st, x, perm, rmax, xp, M, K, p.g.kc)
  if (bits == 4) {
    if (perm) MIQ_F32_STAGE(4, true); else MIQ_F32_STAGE(4, false);
  } else {
    if (perm) MIQ_F32_STAGE(8, true); else MIQ_F32_STAGE(8, false);
  }
#undef MIQ_F32_STAGE
  rc = check_launch("gptq_gemm_f32x staging");
  if (rc) return rc;
  rc = bits == 4 ? gemm_dispatch<4>(p.g, xp, qweight, qzeros, scales, scales_dtype, nullptr, y2, MIQ_F32, workspace,
                                    2 * M, K, N, gs, zero_offset, st)
                 : gemm_dispatch<8>(p.g, xp, qweight, qzeros, scales, scales_dtype, nullptr, y2, MIQ_F32, workspace,
                                    2 * M, K, N, gs, zero_offset, st);
  if (rc) return rc;
  const dim3 g((N / 4 + 255) / 256, M);
  if (out_dtype == MIQ_F16)
    hipLaunchKernelGGL(combine_rows_kernel<__half>, g, dim3(256), 0, st, y2, rmax, bias, static_cast<__half*>(out), M, N);
  else
    hipLaunchKernelGGL(combine_rows_kernel<float>, g, dim3(256), 0, st, y2, rmax, bias, static_cast<float*>(out), M, N);
  return check_launch("gptq_gemm_f32x combine");
}

extern "C" int miq_gptq_gemm_workspace(int M, int K, int N, int gs, int bits, size_t* bytes) {
  MIQ_REQUIRE(bytes, MIQ_ERR_INVALID, "gptq_gemm_workspace: null output");
  *bytes = 0;
  int rc = check_gptq_dims("gptq_gemm_workspace", K, N, gs, bits);
  if (rc) return rc;
  MIQ_REQUIRE(M >= 0, MIQ_ERR_INVALID, "gptq_gemm_workspace: M=%d", M);
  if (M == 0) return MIQ_OK;
  GemmPlan p;
  rc = gemm_plan(M, K, N, gs, bits, &p);
  if (rc) return rc;
  *bytes = p.ws_bytes;
  // the few-row kernel's needs, with or without act-order (the caller may pass either)
  const size_t s0 = gemm_small_workspace(M, K, N, gs, bits, false), s1 = gemm_small_workspace(M, K, N, gs, bits, true);
  if (s0 != SIZE_MAX) *bytes = std::max(*bytes, s0);
  if (s1 != SIZE_MAX) *bytes = std::max(*bytes, s1);
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
  MIQ_REQUIRE(N % 4 == 0 && K % 32 == 0 && aligned(qweight, 16) && aligned(x, 16) && aligned(scales, 4) &&
                  (!perm || aligned(perm, 16)),
              MIQ_ERR_ALIGN, "gptq_gemm: x, qweight and perm must be 16-byte aligned, N %% 4 == 0, K %% 32 == 0");
  MIQ_REQUIRE(scales_dtype == MIQ_F16 || scales_dtype == MIQ_F32, MIQ_ERR_UNSUPPORTED, "gptq_gemm: scales dtype");
  MIQ_REQUIRE(out_dtype == MIQ_F16 || out_dtype == MIQ_F32, MIQ_ERR_UNSUPPORTED, "gptq_gemm: out dtype");
  MIQ_REQUIRE(zero_offset == (float)(int)zero_offset && zero_offset >= 0.f && zero_offset <= 8.f, MIQ_ERR_UNSUPPORTED,
              "gptq_gemm: zero_offset %g (the exact fp16 path takes a small integer)", zero_offset);
  MIQ_REQUIRE(!perm || K <= 32768, MIQ_ERR_UNSUPPORTED, "gptq_gemm: act-order with K=%d > 32768", K);
  hipStream_t st = static_cast<hipStream_t>(stream);
  const __half* xin = static_cast<const __half*>(x);
  // a few rows: the matrix-core kernel that streams the weights like the GEMV
  const size_t need_small = gemm_small_workspace(M, K, N, gs, bits, perm != nullptr);
  if (need_small != SIZE_MAX &&
      (need_small == 0 || (workspace && workspace_bytes >= need_small && aligned(workspace, 256)))) {
    __half* xg = nullptr;
    if (perm) {
      xg = reinterpret_cast<__half*>(static_cast<char*>(workspace) + kCounterBytes);
      rc = stage_rows<4>(xin, perm, xg, M, K, 128, st);
      if (rc) return rc;
    }
    rc = gemm_small(xin, xg, qweight, qzeros, scales, scales_dtype, bias, out, out_dtype, M, K, N, gs, bits,
                    zero_offset, workspace, workspace_bytes, st);
    if (rc != MIQ_ERR_UNSUPPORTED) return rc;
  }
  GemmPlan p;
  rc = gemm_plan(M, K, N, gs, bits, &p);
  if (rc) return rc;
  MIQ_REQUIRE(workspace && workspace_bytes >= p.ws_bytes && aligned(workspace, 256), MIQ_ERR_INVALID,
              "gptq_gemm: workspace of %zu bytes (256-byte aligned) needed, %zu given", p.ws_bytes, workspace_bytes);
  __half* xp = reinterpret_cast<__half*>(static_cast<char*>(workspace) + kCounterBytes + p.partial_bytes);
  rc = bits == 4 ? stage_rows<4>(xin, perm, xp, M, K, p.kc, st) : stage_rows<8>(xin, perm, xp, M, K, p.kc, st);
  if (rc) return rc;
  if (bits == 4)
    return gemm_dispatch<4>(p, xp, qweight, qzeros, scales, scales_dtype, bias, out, out_dtype, workspace, M, K, N, gs,
                            zero_offset, st);
  return gemm_dispatch<8>(p, xp, qweight, qzeros, scales, scales_dtype, bias, out, out_dtype, workspace, M, K, N, gs,
                          zero_offset, st);
}
