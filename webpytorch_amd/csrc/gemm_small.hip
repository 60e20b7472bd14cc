// Int4 GPTQ product for a few rows (M <= 16) of fp16 activations on the gfx950 matrix cores:
// the prefill of a short prompt, a small batch of decode rows. Such a product moves the whole
// weight matrix for little arithmetic, so it is laid out like the one-row GEMV (gemv_mma.hip):
// every wave issues the loads of all its codes, scales and zeros at entry, and the matrix cores
// only have to keep up with HBM.
//
// y[m][n] = sum_k x[m][k] W[k][n] (+ bias), W[k][n] = s[g][n] (q[k][n] - (z[g][n] + zoff)).
//
// Grid (tiles of 64 columns, K-slices); a 256-thread workgroup holds 4 waves that share the 64
// columns and split the workgroup's 4 SPQ steps of 32 k (wave w takes SPQ consecutive steps).
// Lane l loads 16 bytes (4 adjacent columns 4 (l & 15) .. + 3) of packed row l >> 4 of each
// step and feeds them to four MFMAs (v_mfma_f32_16x16x32_f16), MFMA t taking column
// 4 (l & 15) + t: lane l's B fragment of MFMA t is column t of its word, k 8 (l >> 4) .. + 7.
//
// Exact arithmetic. The B fragment is the 8 integers q - (z + zoff) as fp16 (exact: |.| <= 23),
// built without a conversion per value (miq_common.h: b_fragment); A is the fp16 rows of x
// themselves, one 16-row block (rows past M are zero). fp16 x fp16 products are exact in fp32,
// the MFMA sums them in fp32, and the group scale multiplies each group's sums:
// acc += s_g * D. D rows are x rows: lane l holds rows 4 (l >> 4) .. + 3 of its 4 columns.
// Activations are staged in LDS in the pair order of the B halves (k 0, 4, 1, 5, 2, 6, 3, 7).
//
// Reduction. The 4 waves' sums meet in LDS (wave order, deterministic), each wave then finishing
// a quarter of the outputs. With one K-slice it writes y; with several, each output's slices
// meet in a fixed-point word of the workspace's zeroed counter region (mma_tile.h: fix_add),
// whose last arrival writes y.
//
// x is read as fp16 rows (row-major), or, for act-order weights (rows stored by group), from the
// copy the prefill GEMM's gather pass makes (pair order, stage-major with 128-wide stages).
#include <algorithm>

#include "miq_common.h"
#include "mma_tile.h"

namespace miq {
namespace gs {

using namespace mt;

constexpr int kGsTargetWgs = 512;     // split K until the grid has this many workgroups
constexpr int kGsWideMinTiles = 128;  // from this many column tiles, 16 waves cover all of K

constexpr int kXkc = 128;  // stage width of the gathered copy

// 8 fp16 in k order (words (h0,h1) (h2,h3) (h4,h5) (h6,h7)) into pair order (h0,h4) (h1,h5)
// (h2,h6) (h3,h7): k 0, 4, 1, 5, 2, 6, 3, 7, the order of the B halves
__device__ __forceinline__ uint4 pair_order(uint4 v) {
  return make_uint4((v.x & 0xFFFFu) | (v.z << 16), (v.x >> 16) | (v.z & 0xFFFF0000u), (v.y & 0xFFFFu) | (v.w << 16),
                    (v.y >> 16) | (v.w & 0xFFFF0000u));
}

template <int NWV, int SPQ, bool XP, typename ST, typename OT>
__global__ __launch_bounds__(NWV * 64) void gemm_small_kernel(const __half* __restrict__ x,
                                                              const uint32_t* __restrict__ qw,
                                                              const uint32_t* __restrict__ qz,
                                                              const ST* __restrict__ sc,
                                                              const float* __restrict__ bias, OT* __restrict__ out,
                                                              unsigned long long* __restrict__ fixacc,
                                                              float* __restrict__ side, int M, int K, int N,
                                                              float zoff) {
  using SV = typename Scales4<ST>::T;
  constexpr int NT = NWV * 64;         // threads
  constexpr int NG = SPQ / 4;          // groups per wave
  constexpr int WS = NWV * SPQ;        // steps per workgroup
  constexpr int XCH = 16 * WS * 4 / NT;  // 8-wide x chunks staged per thread (= SPQ)
  static_assert(XCH * NT == 16 * WS * 4, "whole chunks");
  __shared__ __align__(16) unsigned char xa[WS * 1024];  // per step: 4 k-chunks x 16 rows x 16 B

  const int tile = blockIdx.x, sl = blockIdx.y, kslices = gridDim.y;
  const int wave = uniform(threadIdx.x >> 6), lane = threadIdx.x & 63;
  const int wst0 = sl * WS;                      // first step of the workgroup
  const int nws = min(WS, K / 32 - wst0);        // its steps: a multiple of 4, > 0
  const int ns = min(SPQ, nws - wave * SPQ);     // this wave's steps (<= 0: none)
  const int st0 = wst0 + wave * SPQ;
  const int c = tile * 64 + (lane & 15) * 4;
  const int cl = min(c, N - 4);                  // loads stay in bounds past N

  // the x chunks first: chunk q = tid + 256 j is (row m, step, k-chunk kc), row fastest, so a
  // wave's LDS stores are 64 consecutive 16-byte slots; rows past M load row M - 1, stage zeros
  uint4 xr[XCH];
#pragma unroll
  for (int j = 0; j < XCH; ++j) {
    const int q = (int)threadIdx.x + NT * j;
    const int m = min(q & 15, M - 1), kc = (q >> 4) & 3, step = q >> 6;
    const int k = min(wst0 + step, wst0 + nws - 1) * 32 + kc * 8;
    const __half* src = XP ? x + ((size_t)(k / kXkc) * M + m) * kXkc + k % kXkc : x + (size_t)m * K + k;
    xr[j] = *reinterpret_cast<const uint4*>(src);
  }
  // every step's codes and every group's scales and zeros of this wave; steps past the
  // workgroup's end reload its last step (a select, not a branch)
  uint4 w[SPQ];
  SV sv[NG];
  uint32_t zw[NG];
#pragma unroll
  for (int i = 0; i < SPQ; ++i) {
    const int s = min(st0 + i, wst0 + nws - 1);
    w[i] = *reinterpret_cast<const uint4*>(qw + (size_t)(4 * s + (lane >> 4)) * N + cl);
  }
#pragma unroll
  for (int gi = 0; gi < NG; ++gi) {
    const int g = min(st0 + 4 * gi, wst0 + nws - 4) >> 2;  // 4 steps per group of 128
    sv[gi] = Scales4<ST>::load(sc + (size_t)g * N + cl);
    zw[gi] = qz[(size_t)g * (N >> 3) + (cl >> 3)];
  }
  __builtin_amdgcn_sched_barrier(0);  // the scheduler keeps every load above the stores below

#pragma unroll
  for (int j = 0; j < XCH; ++j) {
    const int q = (int)threadIdx.x + NT * j;
    const int m = q & 15, step = q >> 6;
    const uint4 pw = (m < M && step < nws) ? (XP ? xr[j] : pair_order(xr[j])) : make_uint4(0u, 0u, 0u, 0u);
    *reinterpret_cast<uint4*>(xa + (size_t)q * 16) = pw;  // step * 1024 + kc * 256 + m * 16
  }
  __syncthreads();

  // this wave's steps: 4 MFMA chains per group, folded with the group scale
  float4v acc[4];
#pragma unroll
  for (int t = 0; t < 4; ++t) acc[t] = (float4v){0.f, 0.f, 0.f, 0.f};
  const unsigned char* ap = xa + (wave * SPQ) * 1024 + (lane >> 4) * 256 + (lane & 15) * 16;
  const int zsh = (cl & 7) * 4;
#pragma unroll
  for (int gi = 0; gi < NG; ++gi) {
    if (4 * gi < ns) {
      half2v zl[4], zh[4];
      zero_pairs<4>(zw[gi] >> zsh, zoff, zl, zh);
      float4v d[4];
#pragma unroll
      for (int t = 0; t < 4; ++t) d[t] = (float4v){0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int s4 = 0; s4 < 4; ++s4) {
        const int i = 4 * gi + s4;
        const half8v av = *reinterpret_cast<const half8v*>(ap + i * 1024);
#pragma unroll
        for (int t = 0; t < 4; ++t)
          d[t] = __builtin_amdgcn_mfma_f32_16x16x32_f16(av, b_fragment<4>(&w[i], t, zl[t], zh[t]), d[t], 0, 0, 0);
      }
#pragma unroll
      for (int t = 0; t < 4; ++t) {
        const float st = Scales4<ST>::get(sv[gi], t);
#pragma unroll
        for (int r = 0; r < 4; ++r) acc[t][r] = fmaf(st, d[t][r], acc[t][r]);
      }
    }
  }

  // the waves' sums in wave order (LDS of A is free once every wave is past its MFMAs)
  __syncthreads();
  float* red = reinterpret_cast<float*>(xa);  // [wave][16][64]
  static_assert(NWV * 16 * 64 * 4 <= WS * 1024, "reduction fits the A buffer");
  constexpr int NV = 16;                      // outputs per lane: v = t * 4 + r
#pragma unroll
  for (int t = 0; t < 4; ++t)
#pragma unroll
    for (int r = 0; r < 4; ++r) red[(wave * NV + t * 4 + r) * 64 + lane] = acc[t][r];
  __syncthreads();
  // each wave finishes NV / NWV of the lane's outputs (returning atomics of one wave complete
  // one after another, so they are spread over the waves)
  constexpr int NW = NV / NWV;
  float ys[NW];
#pragma unroll
  for (int u = 0; u < NW; ++u) {
    const int v = wave * NW + u;
    float y = red[v * 64 + lane];
#pragma unroll
    for (int ww = 1; ww < NWV; ++ww) y += red[(ww * NV + v) * 64 + lane];
    ys[u] = y;
  }
  // output v = t * 4 + r is row 4 (lane >> 4) + r, column c + t
  auto row_of = [&](int v) { return 4 * (lane >> 4) + (v & 3); };
  auto col_of = [&](int v) { return c + (v >> 2); };
  if (kslices == 1) {
#pragma unroll
    for (int u = 0; u < NW; ++u) {
      const int v = wave * NW + u, m = row_of(v), n = col_of(v);
      if (m < M && n < N) out[(size_t)m * N + n] = from_f32<OT>(bias ? ys[u] + bias[n] : ys[u]);
    }
    return;
  }
  // every atomic first, then the checks: the round trips overlap. The words of a tile are laid
  // out [v][lane], so one atomic instruction covers 512 contiguous bytes.
  const size_t w0 = (size_t)tile * NV * 64 + lane, nwords = (size_t)gridDim.x * NV * 64;
  unsigned long long add[NW], old[NW];
#pragma unroll
  for (int u = 0; u < NW; ++u) {
    const int v = wave * NW + u, m = row_of(v), n = col_of(v);
    add[u] = fix_word(ys[u]);
    old[u] = 0;
    if (m < M && n < N)
      old[u] = fix_issue(fixacc + w0 + v * 64, add[u], ys[u], fix_esc(fixacc, w0 + v * 64, side, nwords), sl);
  }
#pragma unroll
  for (int u = 0; u < NW; ++u) {
    const int v = wave * NW + u, m = row_of(v), n = col_of(v);
    float r;
    if (m < M && n < N &&
        fix_finish(fixacc + w0 + v * 64, old[u], add[u], kslices, fix_esc(fixacc, w0 + v * 64, side, nwords), &r))
      out[(size_t)m * N + n] = from_f32<OT>(bias ? r + bias[n] : r);
  }
}

struct Plan {
  int nwv, spq, tiles, kslices;
};

// Either 16 waves per workgroup covering all of K (no split: K <= 16 x 8 steps, and enough
// 64-column tiles to occupy the chip), or 4 waves per workgroup with SPQ (steps per wave) the
// largest whose grid still has ~a workgroup per CU. K-slices beyond one need a fixed-point word
// per output ([tile][16][64] words).
static bool plan(int M, int K, int N, Plan* p) {
  if (M < 1 || M > 16 || K % 128 || N % 8) return false;
  const int steps = K / 32;
  p->tiles = (N + 63) / 64;
  if (p->tiles >= kGsWideMinTiles && steps <= 16 * 8) {  // LDS: 1 KB of A per step
    p->nwv = 16;
    p->spq = steps <= 16 * 4 ? 4 : 8;
    p->kslices = 1;
    return true;
  }
  p->nwv = 4;
  const int cands[3] = {16, 8, 4};
  p->spq = 4;
  for (int i = 0; i < 3; ++i) {
    const int s = cands[i];
    if ((long)p->tiles * ((steps + 4 * s - 1) / (4 * s)) >= kGsTargetWgs) {
      p->spq = s;
      break;
    }
  }
  p->kslices = (steps + 4 * p->spq - 1) / (4 * p->spq);
  if (p->kslices > kFixMaxSlices) return false;
  if (p->kslices > 1 && (size_t)p->tiles * 16 * 64 > kFixMaxWords) return false;
  return true;
}

template <int NWV, int SPQ, bool XP>
static void launch3(const Plan& pl, const __half* x, const int32_t* qw, const int32_t* qz, const void* sc, int sd,
                    const float* bias, void* out, int od, unsigned long long* fixacc, float* side, int M, int K, int N,
                    float zoff, hipStream_t st) {
  const dim3 grid(pl.tiles, pl.kslices);
  const uint32_t* w = reinterpret_cast<const uint32_t*>(qw);
  const uint32_t* z = reinterpret_cast<const uint32_t*>(qz);
#define MIQ_GS_LAUNCH(ST, OT)                                                                                      \
  hipLaunchKernelGGL((gemm_small_kernel<NWV, SPQ, XP, ST, OT>), grid, dim3(NWV * 64), 0, st, x, w, z,            \
                     static_cast<const ST*>(sc), bias, static_cast<OT*>(out), fixacc, side, M, K, N, zoff)
  if (sd == MIQ_F16) {
    if (od == MIQ_F16) MIQ_GS_LAUNCH(__half, __half);
    else MIQ_GS_LAUNCH(__half, float);
  } else {
    if (od == MIQ_F16) MIQ_GS_LAUNCH(float, __half);
    else MIQ_GS_LAUNCH(float, float);
  }
#undef MIQ_GS_LAUNCH
}

}  // namespace gs

// Bytes of the gathered copy of x (act-order) that follows the counter region.
static size_t xg_bytes(int M, int K) { return ((size_t)M * K * 2 + 255) & ~(size_t)255; }

// Bytes of workspace gemm_small needs (0: none; SIZE_MAX: the shape is not covered): the counter
// region, with perm the gathered copy of x, and with several K-slices the escape slots of the
// fixed-point words ([kslices][words] floats).
size_t gemm_small_workspace(int M, int K, int N, int gs_, int bits, bool perm) {
  gs::Plan pl;
  if (bits != 4 || gs_ != 128 || !gs::plan(M, K, N, &pl)) return SIZE_MAX;
  const size_t esc = pl.kslices > 1 ? (size_t)pl.kslices * pl.tiles * 16 * 64 * 4 : 0;
  if (!perm) return pl.kslices > 1 ? kCounterBytes + esc : 0;
  return kCounterBytes + xg_bytes(M, K) + esc;
}

// Launches the few-row product when it covers the shape; MIQ_ERR_UNSUPPORTED (before launching
// anything) otherwise. xg is the gathered copy of x (act-order) or null.
int gemm_small(const __half* x, const __half* xg, const int32_t* qw, const int32_t* qz, const void* sc, int sd,
               const float* bias, void* out, int od, int M, int K, int N, int gs_, int bits, float zoff, void* ws,
               size_t ws_bytes, hipStream_t st) {
  gs::Plan pl;
  if (bits != 4 || gs_ != 128 || !gs::plan(M, K, N, &pl) || !aligned(qw, 16) || !aligned(sc, 16) ||
      !aligned(x, 16))
    return MIQ_ERR_UNSUPPORTED;
  if (pl.kslices > 1 && (!ws || ws_bytes < gemm_small_workspace(M, K, N, gs_, bits, xg != nullptr)))
    return MIQ_ERR_UNSUPPORTED;
  unsigned long long* fixacc = pl.kslices > 1 ? static_cast<unsigned long long*>(ws) : nullptr;
  float* side = pl.kslices > 1 ? reinterpret_cast<float*>(static_cast<char*>(ws) + kCounterBytes +
                                                          (xg ? xg_bytes(M, K) : 0))
                               : nullptr;
  const __half* src = xg ? xg : x;
#define MIQ_GS_CASE(NWV, SPQ)                                                                                      \
  if (pl.nwv == NWV && pl.spq == SPQ) {                                                                            \
    if (xg) gs::launch3<NWV, SPQ, true>(pl, src, qw, qz, sc, sd, bias, out, od, fixacc, side, M, K, N, zoff, st); \
    else gs::launch3<NWV, SPQ, false>(pl, src, qw, qz, sc, sd, bias, out, od, fixacc, side, M, K, N, zoff, st);   \
    return check_launch("gemm_small");                                                                             \
  }
  MIQ_GS_CASE(4, 16) MIQ_GS_CASE(4, 8) MIQ_GS_CASE(4, 4) MIQ_GS_CASE(16, 8) MIQ_GS_CASE(16, 4)
#undef MIQ_GS_CASE
  return MIQ_ERR_UNSUPPORTED;
}

}  // namespace miq
