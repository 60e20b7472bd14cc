// One-row int4 GPTQ GEMV on the gfx950 matrix cores, for layers large enough to be bound by
// HBM bandwidth (the decode projections of 1B+ models, tied heads).
//
// y[n] = sum_k x[k] W[k][n] (+ bias), W[k][n] = s[g][n] (q[k][n] - (z[g][n] + zoff)).
//
// Grid (tiles of 256 columns, K-slices); a 256-thread workgroup holds 4 waves, one per 64
// columns, each taking every 32-k step of its K-slice. For K of 4 to 12 groups the grid is
// instead tiles of 64 columns with the whole K: the four waves take a quarter of the groups
// each and add their partials through LDS, so no reduction crosses workgroups (WS). A wave issues the loads of all its steps
// (16 bytes of codes per lane per step, scales and zeros per group) at entry, then the
// workgroup stages its slice of x in LDS as four int8 digit rows per 64-k step (30-bit fixed
// point at the step's own scale, the int8 digit tile of mma_tile.h) and the waves run four
// v_mfma_i32_16x16x64_i8 per 64-k step that share its A fragment, the codes entering as int8.
// With one K-slice the workgroup writes y. With several, the slices of a column meet
// in one 64-bit word of the workspace's zeroed counter region: each adds its partial as a
// fixed-point integer (2^-24 resolution, offset to stay non-negative) together with a count in
// the top bits, by one agent-scope atomic whose return value tells the last slice that it is
// last and holds the whole sum; that slice writes y (+ bias) and re-zeroes the word. Integer
// sums do not depend on the order of arrival, so results are deterministic, and the reduction
// costs one round trip to the coherence point. Partials the fixed point cannot hold (NaN, Inf,
// |p| >= 2^22) reach the last slice exactly through escape slots (mma_tile.h). Layers with more columns than the counter region
// has words use fp32 partials and a per-tile arrival counter instead (three round trips). Several
// workgroups per CU keep ~50-100 KB of weights in flight per CU.
//
// Input transforms (XM) for the decode step's fused launches, applied while x is staged:
// RMSNorm (1): x * w is staged, every workgroup computes the row's mean square over all K from
// loads issued ahead of its weights, and each slice's partial is divided by
// r = sqrt(mean(x^2) + eps) before it is summed (RMSNorm(x) @ W = ((x * w) @ W) / r, r one
// scalar per row); SwiGLU (2): x is a [gate | up] row of 2K values and silu(gate) * up is staged.
#include <algorithm>

#include "miq_common.h"
#include "mma_tile.h"

namespace miq {
namespace gm {

using namespace mt;

constexpr int kThreadsG = 256;
constexpr int kMaxSlices = kFixMaxSlices;
constexpr size_t kMaxFixCols = kFixMaxWords;

// Groups of 128 values (4 steps of 32). A 256-thread workgroup covers 256 columns; wave w takes
// the 64 columns [64 w, 64 w + 64) and every step of the workgroup's K-slice. Lane l loads 16
// bytes -- the codes of 4 adjacent columns 4 (l & 15) .. + 3 -- of packed row (l >> 4) of each
// step (a wave load covers 4 rows x 256 contiguous bytes), and feeds them to four MFMAs that
// share the step's A fragment: MFMA t's column l & 15 is the lane's column 4 (l & 15) + t. Each
// lane thus holds whole column results for 4 columns; no reduction across waves is needed.
constexpr int kGmDepth = 4;  // steps of codes in flight per wave (0: all of the slice, issued at entry)
constexpr int kNormLoads = 8;  // float4 loads per thread of an RMSNorm row issued up front (K <= 8192)

template <typename XT, typename ST, typename OT, int SPQ, bool PERM, int XM, bool WS>
__global__ __launch_bounds__(kThreadsG) void gemv_mma_kernel(const XT* __restrict__ x, const int32_t* __restrict__ perm,
                                                             const uint32_t* __restrict__ qw,
                                                             const uint32_t* __restrict__ qz, const ST* __restrict__ sc,
                                                             const float* __restrict__ bias, OT* __restrict__ out,
                                                             float* __restrict__ partials, int* __restrict__ counters,
                                                             unsigned long long* __restrict__ fixacc, int K, int N,
                                                             float zoff, int slice_steps, const float* __restrict__ nw,
                                                             float eps) {
  static_assert(XM == 0 || (sizeof(XT) == 4 && !PERM), "input transforms take fp32 rows in k order");
  constexpr int NG = SPQ / 4;            // groups per wave
  constexpr int XS = WS ? 4 * SPQ : SPQ;  // staged steps per workgroup
  using SV = typename Scales4<ST>::T;
  __shared__ __align__(16) unsigned char xa[(XS / 2) * kStep8Bytes];
  __shared__ float2 cx[XS];
  __shared__ int is_last;
  __shared__ float ssw[kThreadsG / 64];
  __shared__ float wsum[WS ? kThreadsG : 1];
  const int tile = blockIdx.x, sl = blockIdx.y, kslices = gridDim.y;
  const int wave = uniform(threadIdx.x >> 6), lane = threadIdx.x & 63;
  const int st0 = sl * slice_steps;
  const int ns = min(slice_steps, K / 32 - st0);  // the workgroup's steps: a multiple of 4, > 0 by the planner
  // WS: the four waves share the tile's 64 columns and split the slice's groups (the first
  // waves one group fewer when they do not divide); else each wave takes 64 of 256 columns
  const int gw0 = WS ? wave * (ns / 4) / 4 : 0, gw1 = WS ? (wave + 1) * (ns / 4) / 4 : ns / 4;
  const int wns = 4 * (gw1 - gw0);               // this wave's steps (> 0: the planner gives WS >= 4 groups)
  const int rb = (st0 + 4 * gw0) * 4;            // first packed row of the wave's steps
  const int c = WS ? tile * 64 + (lane & 15) * 4 : tile * 256 + wave * 64 + (lane & 15) * 4;
  const int cl = min(c, N - 4);                    // loads stay in bounds past N
  // this thread's 8 activations of the slice (or their permutation indices) as raw 16-byte
  // loads, issued before the weights; gathering and converting wait until the weight loads are
  // in flight, so the activation round trip overlaps them. Threads past the slice's chunks
  // stage one of the first four steps' chunks again (same values to the same LDS words): with
  // no branch around them, the compiler keeps the loads ahead of the weight loads.
  const int ch = (int)threadIdx.x < ns * 4 ? (int)threadIdx.x : (int)(threadIdx.x & 15);
  const int k0 = st0 * 32 + ch * 8;
  const uint4* src = PERM ? reinterpret_cast<const uint4*>(perm + k0) : reinterpret_cast<const uint4*>(x + k0);
  const uint4 xr0 = src[0];
  const uint4 xr1 = src[(PERM || sizeof(XT) == 4) ? 1 : 0];
  uint4 ur0, ur1;  // SwiGLU: the up half of the chunk
  if constexpr (XM == 2) {
    const uint4* usrc = reinterpret_cast<const uint4*>(reinterpret_cast<const float*>(x) + K + k0);
    ur0 = usrc[0];
    ur1 = usrc[1];
  }
  float4 xf[kNormLoads];  // RMSNorm: the whole row, for its mean square (clamped loads, masked below)
  if constexpr (XM == 1) {
    const float4* xq = reinterpret_cast<const float4*>(x);
#pragma unroll
    for (int j = 0; j < kNormLoads; ++j) xf[j] = xq[min((int)threadIdx.x + j * kThreadsG, K / 4 - 1)];
  }
  // every step's codes and every group's scales and zeros of this wave, issued up front
  uint4 w[SPQ];
  SV sv[NG];
  uint32_t zw[NG];
  const uint32_t* wp = qw + (size_t)(rb + (lane >> 4)) * N + cl;
  // steps past the slice's end reload its last step (a select, not a branch: a branch around a
  // load makes the compiler's wait counts conservative at the join)
  auto wload = [&](int i) __attribute__((always_inline)) {
    return *reinterpret_cast<const uint4*>(wp + (size_t)(4 * min(i, wns - 1)) * N);
  };
  // the scales and zeros first (the first group's fold needs them), then the codes of the first
  // DEPTH steps; each group issues the codes DEPTH steps ahead of it
  constexpr int DEPTH = (kGmDepth > 0 && kGmDepth < SPQ) ? kGmDepth : SPQ;
#pragma unroll
  for (int gi = 0; gi < NG; ++gi) {
    const int g = (rb >> 4) + min(gi, (wns >> 2) - 1);  // 16 packed rows per group
    sv[gi] = Scales4<ST>::load(sc + (size_t)g * N + cl);
    zw[gi] = qz[(size_t)g * (N >> 3) + (cl >> 3)];
  }
#pragma unroll
  for (int i = 0; i < DEPTH; ++i) w[i] = wload(i);
  __builtin_amdgcn_sched_barrier(0);  // the scheduler keeps every load above the conversions
  float v[8];
  const uint32_t r[8] = {xr0.x, xr0.y, xr0.z, xr0.w, xr1.x, xr1.y, xr1.z, xr1.w};
  if (PERM) {
#pragma unroll
    for (int j = 0; j < 8; ++j) v[j] = to_f32(x[r[j]]);  // indices are non-negative
  } else if (sizeof(XT) == 2) {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      v[2 * j] = __half2float(__ushort_as_half((unsigned short)(r[j] & 0xFFFFu)));
      v[2 * j + 1] = __half2float(__ushort_as_half((unsigned short)(r[j] >> 16)));
    }
  } else {
#pragma unroll
    for (int j = 0; j < 8; ++j) v[j] = __uint_as_float(r[j]);
  }
  if constexpr (XM == 1) {
    float ss = 0.f;
#pragma unroll
    for (int j = 0; j < kNormLoads; ++j)
      if ((int)threadIdx.x + j * kThreadsG < K / 4)
        ss += xf[j].x * xf[j].x + xf[j].y * xf[j].y + xf[j].z * xf[j].z + xf[j].w * xf[j].w;
    const float4* xq = reinterpret_cast<const float4*>(x);
    for (int i = threadIdx.x + kNormLoads * kThreadsG; i < K / 4; i += kThreadsG) {
      const float4 t = xq[i];
      ss += t.x * t.x + t.y * t.y + t.z * t.z + t.w * t.w;
    }
    ss = wave_sum(ss);
    if (lane == 0) ssw[wave] = ss;
    const float4 w0 = reinterpret_cast<const float4*>(nw + k0)[0], w1 = reinterpret_cast<const float4*>(nw + k0)[1];
    const float wv[8] = {w0.x, w0.y, w0.z, w0.w, w1.x, w1.y, w1.z, w1.w};
#pragma unroll
    for (int j = 0; j < 8; ++j) v[j] = v[j] * wv[j];
  } else if constexpr (XM == 2) {
    const uint32_t u[8] = {ur0.x, ur0.y, ur0.z, ur0.w, ur1.x, ur1.y, ur1.z, ur1.w};
#pragma unroll
    for (int j = 0; j < 8; ++j) v[j] = (v[j] * (1.f / (1.f + expf(-v[j])))) * __uint_as_float(u[j]);
  }
  stage_digits(ch, v, xa, cx);
  __syncthreads();
  float rn = 1.f;  // RMSNorm: r of the row (the same value in every workgroup)
  if constexpr (XM == 1) rn = sqrtf((((ssw[0] + ssw[1]) + ssw[2]) + ssw[3]) / (float)K + eps);
  // A rows 0-3 (the digits) are read by lanes 0-3 of each 16; the other rows of D are never used
  const bool arow = (lane & 15) < 4;
  uint32_t mk = 0x0F0F0F0Fu;
  asm volatile("" : "+v"(mk));
  const unsigned char* ap = xa + (lane >> 4) * 64 + (lane & 15) * 16 + (size_t)(2 * gw0) * kStep8Bytes;
  const float2* cw = cx + 2 * gw0;  // the wave's 64-k steps among the staged ones
  const int zsh = (cl & 7) * 4;
  float acc[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int gi = 0; gi < NG; ++gi) {
    if constexpr (DEPTH < SPQ) {
      if (4 * gi + DEPTH < SPQ) {
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int s4 = 0; s4 < 4; ++s4) w[4 * gi + DEPTH + s4] = wload(4 * gi + DEPTH + s4);
        __builtin_amdgcn_sched_barrier(0);
      }
    }
    if (4 * gi < wns) {
      float pg[4] = {0.f, 0.f, 0.f, 0.f};
      float xs = 0.f;
#pragma unroll
      for (int h = 0; h < 2; ++h) {  // the group's two 64-k steps
        const int j = 2 * gi + h;
        i32x4 av = {0, 0, 0, 0};
        if (arow) av = *reinterpret_cast<const i32x4*>(ap + j * kStep8Bytes);
        const float2 cxj = cw[j];
        xs += cxj.y;
        const uint32_t qa[4] = {w[2 * j].x, w[2 * j].y, w[2 * j].z, w[2 * j].w};
        const uint32_t qb[4] = {w[2 * j + 1].x, w[2 * j + 1].y, w[2 * j + 1].z, w[2 * j + 1].w};
        i32x4 dq[4];
#pragma unroll
        for (int t = 0; t < 4; ++t) {
          const i32x4 b = {(int)(qa[t] & mk), (int)((qa[t] >> 4) & mk), (int)(qb[t] & mk), (int)((qb[t] >> 4) & mk)};
          dq[t] = __builtin_amdgcn_mfma_i32_16x16x64_i8(av, b, (i32x4){0, 0, 0, 0}, 0, 0, 0);
        }
#pragma unroll
        for (int t = 0; t < 4; ++t) {
          const int lo = dq[t][0] + (dq[t][1] << 8), hi = dq[t][2] + (dq[t][3] << 8);
          pg[t] = fmaf(fmaf((float)hi, 65536.f, (float)lo), cxj.x, pg[t]);
        }
      }
#pragma unroll
      for (int t = 0; t < 4; ++t) {
        const float zc = (float)((zw[gi] >> (zsh + 4 * t)) & 15u) + zoff;
        acc[t] = fmaf(Scales4<ST>::get(sv[gi], t), pg[t] - zc * xs, acc[t]);
      }
    }
  }
  if constexpr (XM == 1) {
#pragma unroll
    for (int t = 0; t < 4; ++t) acc[t] = acc[t] / rn;
  }
  const bool mine = lane < 16 && c < N;
  if constexpr (WS) {  // the waves' partials of the same 64 columns, summed in wave order
    if (lane < 16)
#pragma unroll
      for (int t = 0; t < 4; ++t) wsum[wave * 64 + lane * 4 + t] = acc[t];
    __syncthreads();
    const int n = tile * 64 + (int)threadIdx.x;
    if (threadIdx.x < 64 && n < N) {
      const float y = ((wsum[threadIdx.x] + wsum[64 + threadIdx.x]) + wsum[128 + threadIdx.x]) + wsum[192 + threadIdx.x];
      out[n] = from_f32<OT>(bias ? y + bias[n] : y);
    }
    return;
  }
  if (kslices == 1) {
    if (mine)
#pragma unroll
      for (int t = 0; t < 4; ++t) out[c + t] = from_f32<OT>(bias ? acc[t] + bias[c + t] : acc[t]);
    return;
  }
  if (fixacc) {
    // split K over fixed-point words: lane l takes column 4 (l & 15) + (l >> 4) of the wave's 64
    const int t = lane >> 4;
    const float a0 = __shfl(acc[0], lane & 15, 64), a1 = __shfl(acc[1], lane & 15, 64);
    const float a2 = __shfl(acc[2], lane & 15, 64), a3 = __shfl(acc[3], lane & 15, 64);
    const float p = t == 0 ? a0 : t == 1 ? a1 : t == 2 ? a2 : a3;
    const int n = tile * 256 + wave * 64 + (lane & 15) * 4 + t;
    float y;
    if (n < N && fix_add(fixacc + n, p, kslices, sl, fix_esc(fixacc, n, partials, N), &y))
      out[n] = from_f32<OT>(bias ? y + bias[n] : y);
    return;
  }
  // split K: partials at device scope, the last workgroup of the tile sums them in slice order
  if (mine)
#pragma unroll
    for (int t = 0; t < 4; ++t)
      __hip_atomic_store(partials + (size_t)sl * N + c + t, acc[t], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
  if (threadIdx.x == 0)
    is_last = __hip_atomic_fetch_add(counters + tile, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == kslices - 1;
  __syncthreads();
  if (!is_last) return;
  const int n = tile * 256 + (int)threadIdx.x;
  if (n < N) {
    float pp[kMaxSlices];
#pragma unroll
    for (int i = 0; i < kMaxSlices; ++i)  // all loads in flight at once
      pp[i] = i < kslices ? __hip_atomic_load(partials + (size_t)i * N + n, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT)
                          : 0.f;
    float s = 0.f;
#pragma unroll
    for (int i = 0; i < kMaxSlices; ++i)
      if (i < kslices) s += pp[i];
    out[n] = from_f32<OT>(bias ? s + bias[n] : s);
  }
  if (threadIdx.x == 0) __hip_atomic_store(counters + tile, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Launch shape: K-slices of a multiple of 4 steps (whole groups), at most 24 steps and 32
// slices, chosen by a cost in steps per CU: the workgroups a CU runs (rounded up over the CUs)
// times (slice steps + kWgSteps, the per-workgroup cost of staging and reduction in step units),
// and a quarter more per 8 slice steps when a CU runs a single workgroup (its waves have no
// partner to overlap their loads and arithmetic with); on a tie the longer slice. Measured over
// slice lengths on 12 shapes of the 0.5B and 7B decoders (a one-row activation), this picks the
// fastest or within 2.5% on each; the earlier rule (four workgroups per CU) left 3584 -> 37888
// 12 workgroups over a round (16.6 us at 16 steps against 15.2 us at 24) and 3584 -> 4608 at
// 4 steps (4.5 us against 4.4 at 8). SPQ is the slice length rounded up to an instantiated capacity.
struct Plan {
  int tiles, kslices, slice_steps, spq;
  bool fixed;  // split K reduced in fixed-point words of the counter region
  bool ws;     // 64-column tiles, K split over the workgroup's waves (no reduction across workgroups)
  size_t ws_bytes;
};

constexpr int kWgSteps = 8;

static bool plan(int K, int N, Plan* p) {
  const int steps = K / 32;
  p->tiles = (N + 255) / 256;
  int ss = 0;
  long best = 0;
  for (int c = 4; c <= 24; c += 4) {
    const int ks = (steps + c - 1) / c;
    if (ks <= kMaxSlices) {
      const long per_cu = ((long)p->tiles * ks + kCUs - 1) / kCUs;
      const long cost = per_cu * (c + kWgSteps) * (per_cu == 1 ? 32 + c : 32);
      if (!ss || cost <= best) {
        ss = c;
        best = cost;
      }
    }
    if (c >= steps) break;  // one slice already covers K
  }
  if (!ss) return false;
  p->slice_steps = ss;
  p->kslices = (steps + ss - 1) / ss;
  if (p->kslices > kMaxSlices || (p->kslices > 1 && p->tiles > kMaxCounters)) return false;
  p->spq = ss <= 4 ? 4 : ss <= 8 ? 8 : ss <= 12 ? 12 : ss <= 16 ? 16 : 24;
  p->fixed = p->kslices > 1 && (size_t)N <= kMaxFixCols;
  // K of 4 to 12 groups: 64-column tiles whose four waves split K and add their partials in LDS,
  // with no reduction across workgroups (measured on one-row graphs, us per call: 896 -> 4864
  // 3.51 -> 3.20, 896 -> 1152 3.20 -> 2.92, 896 -> 9728 4.04 -> 3.43, 896 -> 151936 15.5 -> 14.3,
  // 1536 -> 8960 4.21 -> 4.06; at 16 groups the split slices were faster: 2048 -> 8192 4.35
  // against 4.56, 2048 -> 2048 3.35 against 4.04)
  const int groups = steps / 4;
  p->ws = groups >= 4 && groups <= 12;
  if (p->ws) {
    p->tiles = (N + 63) / 64;
    p->kslices = 1;
    p->slice_steps = steps;
    p->spq = 4 * ((groups + 3) / 4);
    p->fixed = false;
  }
  // after the counter region: fp32 partials [kslices][N] (slow path) or the fixed-point
  // words' escape slots, same shape
  p->ws_bytes = p->kslices == 1 ? 0 : kCounterBytes + (size_t)p->kslices * N * 4;
  return true;
}

template <typename XT, typename ST, typename OT, int XM>
static int launch(const Plan& pl, const void* x, const int32_t* perm, const int32_t* qw, const int32_t* qz,
                  const void* sc, const float* bias, void* out, void* ws, int K, int N, float zoff, const float* nw,
                  float eps, hipStream_t st) {
  const bool slow = pl.kslices > 1 && !pl.fixed;
  int* counters = slow ? static_cast<int*>(ws) : nullptr;
  float* partials = pl.kslices > 1 ? reinterpret_cast<float*>(static_cast<char*>(ws) + kCounterBytes) : nullptr;
  unsigned long long* fixacc = pl.fixed ? static_cast<unsigned long long*>(ws) : nullptr;
  dim3 grid(pl.tiles, pl.kslices);
#define MIQ_GM_LAUNCH(S, P)                                                                                        \
  if (pl.ws) {                                                                                                     \
    if constexpr (S <= 16)                                                                                         \
      hipLaunchKernelGGL((gemv_mma_kernel<XT, ST, OT, S, P, XM, true>), grid, dim3(kThreadsG), 0, st,             \
                         static_cast<const XT*>(x), perm, reinterpret_cast<const uint32_t*>(qw),                     \
                         reinterpret_cast<const uint32_t*>(qz), static_cast<const ST*>(sc), bias,                    \
                         static_cast<OT*>(out), partials, counters, fixacc, K, N, zoff, pl.slice_steps, nw, eps);    \
  } else                                                                                                           \
  hipLaunchKernelGGL((gemv_mma_kernel<XT, ST, OT, S, P, XM, false>), grid, dim3(kThreadsG), 0, st,              \
                     static_cast<const XT*>(x), perm, reinterpret_cast<const uint32_t*>(qw),                         \
                     reinterpret_cast<const uint32_t*>(qz), static_cast<const ST*>(sc), bias, static_cast<OT*>(out), \
                     partials, counters, fixacc, K, N, zoff, pl.slice_steps, nw, eps)
#define MIQ_GM_SPQ(S)            \
  {                              \
    if constexpr (XM == 0) {     \
      if (perm)                  \
        MIQ_GM_LAUNCH(S, true);  \
      else                       \
        MIQ_GM_LAUNCH(S, false); \
    } else {                     \
      MIQ_GM_LAUNCH(S, false);   \
    }                            \
  }
  if (pl.spq == 4) MIQ_GM_SPQ(4)
  else if (pl.spq == 8) MIQ_GM_SPQ(8)
  else if (pl.spq == 12) MIQ_GM_SPQ(12)
  else if (pl.spq == 16) MIQ_GM_SPQ(16)
  else MIQ_GM_SPQ(24)
#undef MIQ_GM_SPQ
#undef MIQ_GM_LAUNCH
  return check_launch("gemv_mma");
}

}  // namespace gm

// Entry used by miq_gptq_gemv for one row of int4 codes (see there for the argument contract).
// Returns MIQ_ERR_UNSUPPORTED (before launching anything) for shapes it does not cover.
int gemv_mma(const void* x, int xd, const int32_t* perm, const int32_t* qw, const int32_t* qz, const void* sc,
             int sd, const float* bias, void* out, int od, int K, int N, int gs, float zoff, void* ws,
             size_t ws_bytes, hipStream_t st, int xmode, const float* norm_w, float eps) {
  if (gs != 128 || K % 128 || N % 8 || !aligned(qw, 16) || !aligned(sc, 16) || !aligned(x, 16) ||
      (perm && !aligned(perm, 16)))
    return MIQ_ERR_UNSUPPORTED;
  if (xmode != 0 && (xd != MIQ_F32 || od != MIQ_F32 || perm || (xmode == 1 && (!norm_w || !aligned(norm_w, 16)))))
    return MIQ_ERR_UNSUPPORTED;
  gm::Plan pl;
  if (!gm::plan(K, N, &pl)) return MIQ_ERR_UNSUPPORTED;
  if (pl.kslices > 1 && (!ws || ws_bytes < pl.ws_bytes)) return MIQ_ERR_UNSUPPORTED;
  if (xmode == 1) {
    if (sd == MIQ_F16) return gm::launch<float, __half, float, 1>(pl, x, perm, qw, qz, sc, bias, out, ws, K, N, zoff, norm_w, eps, st);
    return gm::launch<float, float, float, 1>(pl, x, perm, qw, qz, sc, bias, out, ws, K, N, zoff, norm_w, eps, st);
  }
  if (xmode == 2) {
    if (sd == MIQ_F16) return gm::launch<float, __half, float, 2>(pl, x, perm, qw, qz, sc, bias, out, ws, K, N, zoff, nullptr, 0.f, st);
    return gm::launch<float, float, float, 2>(pl, x, perm, qw, qz, sc, bias, out, ws, K, N, zoff, nullptr, 0.f, st);
  }
#define MIQ_GM_TYPES(XT, ST, OT) \
  return gm::launch<XT, ST, OT, 0>(pl, x, perm, qw, qz, sc, bias, out, ws, K, N, zoff, nullptr, 0.f, st)
  if (xd == MIQ_F16) {
    if (sd == MIQ_F16) { if (od == MIQ_F16) MIQ_GM_TYPES(__half, __half, __half); MIQ_GM_TYPES(__half, __half, float); }
    if (od == MIQ_F16) MIQ_GM_TYPES(__half, float, __half);
    MIQ_GM_TYPES(__half, float, float);
  }
  if (sd == MIQ_F16) { if (od == MIQ_F16) MIQ_GM_TYPES(float, __half, __half); MIQ_GM_TYPES(float, __half, float); }
  if (od == MIQ_F16) MIQ_GM_TYPES(float, float, __half);
  MIQ_GM_TYPES(float, float, float);
#undef MIQ_GM_TYPES
}

// Workspace bytes gemv_mma needs for this shape (0 if it needs none or does not cover it).
size_t gemv_mma_workspace(int K, int N) {
  gm::Plan pl;
  if (K % 128 || !gm::plan(K, N, &pl)) return 0;
  return pl.ws_bytes;
}

}  // namespace miq
