// Sparse mixture-of-experts MLP on gfx950: device-side routing, expert-grouped GPTQ GEMMs on the
// matrix cores, and a deterministic combine. No step needs the host, so a decode step with MoE
// layers can be captured in a graph with its routing live.
//
//   route    logits [T][E] fp32 -> float64 softmax -> top-k -> (optional) renormalisation;
//            per token its k experts in ascending order with fp32 weights; per expert the list
//            of its (token, weight) slots in ascending token order ("sorted slots"); and a
//            table of row tiles (expert, first slot, rows) that the GEMMs walk.
//   gate_up  h[slot] = silu(x[token] @ Wg[e]) * (x[token] @ Wu[e])   (fp32, stored as fp16 hi + lo)
//   down     y[slot] = w[slot] * (h[slot] @ Wd[e])                    (fp32)
//   combine  out[t] = sum over t's experts in ascending order of y[slot]  (fp32)
//
// The combine order (experts ascending, starting from zero) and the fp32 weight multiply are the
// reference's (`webtorch/lm_engine.py:294-333`). The GEMMs use the prefill GEMM's exact
// dequantization and MFMA mapping (see gptq_gemm.hip); a workgroup takes one row tile of one
// expert (up to kMoeBM rows) and 256 output columns. The intermediate h keeps fp32 accuracy
// through the fp16 matrix cores as two fp16 halves, hi = fp16(h) and lo = fp16(h - hi)
// (together exact to about 22 bits); the down GEMM multiplies both by the same weights.
#include <type_traits>

#include "miq_common.h"

namespace miq {

constexpr int kMoeBM = 32;      // rows per tile (two 16-row MFMA blocks)
constexpr int kMoeMaxTK = 4096;  // T * k handled by the single-workgroup router

// Offsets (in 4-byte words) of the route buffer's arrays.
struct RouteLayout {
  size_t topk_e, topk_w, slot_of, sorted_tok, sorted_w, expert_off, ntiles, tiles, words;
  int max_tiles;
};

__host__ __device__ inline RouteLayout route_layout(int T, int E, int k) {
  RouteLayout L;
  const size_t tk = (size_t)T * k;
  L.max_tiles = (int)((tk + kMoeBM - 1) / kMoeBM) + E;
  L.topk_e = 0;
  L.topk_w = L.topk_e + tk;
  L.slot_of = L.topk_w + tk;
  L.sorted_tok = L.slot_of + tk;
  L.sorted_w = L.sorted_tok + tk;
  L.expert_off = L.sorted_w + tk;
  L.ntiles = L.expert_off + E + 1;
  L.tiles = (L.ntiles + 1 + 3) & ~(size_t)3;  // 16-byte aligned int4 entries
  L.words = L.tiles + 4 * (size_t)L.max_tiles;
  return L;
}

// ------------------------------------------------------------------------------------
// Router: one workgroup of 1024 threads. Phase 1, a wave per token: float64 softmax over the E
// logits, k rounds of arg-max (lowest index on ties), renormalisation over the picks, then the
// picks sorted by expert. Phase 2: per-expert counts, offsets and row tiles. Phase 3: a thread
// per expert walks the tokens in order and assigns slots, so each expert's rows are in ascending
// token order.
__global__ __launch_bounds__(1024) void moe_route_kernel(const float* __restrict__ logits, int T, int E, int k,
                                                         int norm_topk, int* __restrict__ route) {
  const RouteLayout L = route_layout(T, E, k);
  int* topk_e = route + L.topk_e;
  float* topk_w = reinterpret_cast<float*>(route + L.topk_w);
  int* slot_of = route + L.slot_of;
  int* sorted_tok = route + L.sorted_tok;
  float* sorted_w = reinterpret_cast<float*>(route + L.sorted_w);
  int* expert_off = route + L.expert_off;
  int* ntiles = route + L.ntiles;
  int4* tiles = reinterpret_cast<int4*>(route + L.tiles);

  // everything phases 2 and 3 read lives in LDS
  extern __shared__ int lds_i[];
  int* se = lds_i;                                         // [T*k] chosen experts, ascending per token
  float* sw = reinterpret_cast<float*>(lds_i + T * k);     // [T*k] their weights
  int* cnt = lds_i + 2 * T * k;                            // [E]
  int* off = cnt + E;                                      // [E + 1]
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, nw = blockDim.x >> 6;

  for (int t = wave; t < T; t += nw) {
    const float* lt = logits + (size_t)t * E;
    double mx = -INFINITY;
    for (int e = lane; e < E; e += 64) mx = fmax(mx, (double)lt[e]);
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) mx = fmax(mx, __shfl_xor(mx, o, 64));
    double sum = 0.0;
    for (int e = lane; e < E; e += 64) sum += exp((double)lt[e] - mx);
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) sum += __shfl_xor(sum, o, 64);
    // k rounds of arg-max over p = exp(l - max) / sum; a picked expert is excluded afterwards
    int pick_e[32];
    double pick_p[32];
    double psum = 0.0;
    for (int j = 0; j < k; ++j) {
      double best = -1.0;
      int be = E;
      for (int e = lane; e < E; e += 64) {
        bool taken = false;
        for (int i = 0; i < j; ++i) taken |= (pick_e[i] == e);
        if (taken) continue;
        const double pe = exp((double)lt[e] - mx) / sum;
        if (pe > best || (pe == best && e < be)) { best = pe; be = e; }
      }
#pragma unroll
      for (int o = 32; o > 0; o >>= 1) {
        const double ob = __shfl_xor(best, o, 64);
        const int oe = __shfl_xor(be, o, 64);
        if (ob > best || (ob == best && oe < be)) { best = ob; be = oe; }
      }
      pick_e[j] = be;
      pick_p[j] = best;
      psum += best;
    }
    if (lane == 0) {
      // ascending expert order (insertion sort of k <= 32 picks)
      for (int a = 1; a < k; ++a)
        for (int b = a; b > 0 && pick_e[b - 1] > pick_e[b]; --b) {
          const int te = pick_e[b]; pick_e[b] = pick_e[b - 1]; pick_e[b - 1] = te;
          const double tp = pick_p[b]; pick_p[b] = pick_p[b - 1]; pick_p[b - 1] = tp;
        }
      for (int j = 0; j < k; ++j) {
        const float w = (float)(norm_topk ? pick_p[j] / psum : pick_p[j]);
        se[t * k + j] = pick_e[j];
        sw[t * k + j] = w;
        topk_e[t * k + j] = pick_e[j];
        topk_w[t * k + j] = w;
      }
    }
  }
  for (int e = threadIdx.x; e < E; e += blockDim.x) cnt[e] = 0;
  __syncthreads();
  for (int i = threadIdx.x; i < T * k; i += blockDim.x) atomicAdd(&cnt[se[i]], 1);
  __syncthreads();
  if (threadIdx.x == 0) {
    int o = 0, nt = 0;
    for (int e = 0; e < E; ++e) {
      off[e] = o;
      expert_off[e] = o;
      for (int r0 = 0; r0 < cnt[e]; r0 += kMoeBM) tiles[nt++] = make_int4(e, o + r0, min(kMoeBM, cnt[e] - r0), 0);
      o += cnt[e];
    }
    off[E] = o;
    expert_off[E] = o;
    *ntiles = nt;
  }
  __syncthreads();
  for (int e = threadIdx.x; e < E; e += blockDim.x) {
    int s = off[e];
    for (int t = 0; t < T; ++t)
      for (int j = 0; j < k; ++j)
        if (se[t * k + j] == e) {
          slot_of[t * k + j] = s;
          sorted_tok[s] = t;
          sorted_w[s] = sw[t * k + j];
          ++s;
        }
  }
}

// ------------------------------------------------------------------------------------
// Grouped GEMM over row tiles. GATE_UP: two weight sets sharing the activations, epilogue
// h = silu(g) * u stored as fp16 hi and lo planes. Otherwise (down): one set whose activations
// are those two planes (two MFMAs per weight fragment), epilogue y = w[slot] * acc in fp32.
template <int BITS, int KC, bool GATE_UP, typename ST>
__global__ __launch_bounds__(256) void moe_gemm_kernel(
    const __half* __restrict__ a, const int* __restrict__ route, int T, int E, int k,
    const uint32_t* __restrict__ qw0, const uint32_t* __restrict__ qz0, const ST* __restrict__ sc0,
    const uint32_t* __restrict__ qw1, const uint32_t* __restrict__ qz1, const ST* __restrict__ sc1,
    size_t qw_stride, size_t qz_stride, size_t sc_stride, size_t a_plane, void* __restrict__ out,
    size_t out_plane, int K, int N, int gs, float zoff) {
  constexpr int PER = 32 / BITS;
  constexpr int TM = kMoeBM / 16;
  constexpr int STEPS = KC / 32;
  constexpr int RB = BITS == 4 ? 1 : 2;
  constexpr int NSET = GATE_UP ? 2 : 1;
  constexpr int NA = GATE_UP ? 1 : 2;  // activation planes (down: hi and lo)
  __shared__ __align__(16) _Float16 xs[NA][kMoeBM * KC];

  const RouteLayout L = route_layout(T, E, k);
  const int tile = blockIdx.y;
  if (tile >= route[L.ntiles]) return;  // uniform: fewer tiles than the grid allows
  const int4 td = reinterpret_cast<const int4*>(route + L.tiles)[tile];
  const int e = td.x, slot0 = td.y, nrows = td.z;
  const int* sorted_tok = route + L.sorted_tok;
  const float* sorted_w = reinterpret_cast<const float*>(route + L.sorted_w);

  const int lane = threadIdx.x & 63;
  const int wave = uniform(threadIdx.x >> 6);
  const int p = lane & 15, kb = lane >> 4;
  const int ncol = blockIdx.x * 256 + wave * 64 + 4 * p;
  const bool colok = ncol < N;
  const bool wave_active = blockIdx.x * 256 + wave * 64 < N;
  const int NZ = N / PER;
  const int zshift = (ncol % PER) * BITS;
  const uint32_t* qw[2] = {qw0 + e * qw_stride, GATE_UP ? qw1 + e * qw_stride : nullptr};
  const uint32_t* qz[2] = {qz0 + e * qz_stride, GATE_UP ? qz1 + e * qz_stride : nullptr};
  const ST* sc[2] = {sc0 + e * sc_stride, GATE_UP ? sc1 + e * sc_stride : nullptr};

  float4v acc[NSET][TM][4];
#pragma unroll
  for (int q = 0; q < NSET; ++q)
#pragma unroll
    for (int t = 0; t < TM; ++t)
#pragma unroll
      for (int s = 0; s < 4; ++s) acc[q][t][s] = (float4v){0.f, 0.f, 0.f, 0.f};

  for (int kc0 = 0; kc0 < K; kc0 += KC) {
    uint4 bw[NSET][STEPS][RB];
    uint4 sraw[NSET];
    uint32_t zraw[NSET];
#pragma unroll
    for (int q = 0; q < NSET; ++q) {
      sraw[q] = make_uint4(0u, 0u, 0u, 0u);
      zraw[q] = 0;
#pragma unroll
      for (int st = 0; st < STEPS; ++st)
#pragma unroll
        for (int rb = 0; rb < RB; ++rb) bw[q][st][rb] = make_uint4(0u, 0u, 0u, 0u);
      if (colok) {
#pragma unroll
        for (int st = 0; st < STEPS; ++st)
#pragma unroll
          for (int rb = 0; rb < RB; ++rb) {
            const int row = (kc0 + st * 32) / PER + kb * RB + rb;
            bw[q][st][rb] = *reinterpret_cast<const uint4*>(qw[q] + (size_t)row * N + ncol);
          }
        const int g = kc0 / gs;
        sraw[q] = load_scales4<ST>(sc[q] + (size_t)g * N + ncol);
        zraw[q] = qz[q][(size_t)g * NZ + ncol / PER];
      }
    }
    __syncthreads();
    for (int ci = threadIdx.x; ci < NA * kMoeBM * KC / 8; ci += 256) {
      const int pl = ci / (kMoeBM * KC / 8), cr = ci - pl * (kMoeBM * KC / 8);
      const int r = cr / (KC / 8), kk = (cr - r * (KC / 8)) * 8;
      float v[8];
      if (r < nrows) {
        const size_t src = GATE_UP ? (size_t)sorted_tok[slot0 + r] : (size_t)(slot0 + r);
        load8(a + (size_t)pl * a_plane + src * K + kc0 + kk, v);
      } else {
#pragma unroll
        for (int j = 0; j < 8; ++j) v[j] = 0.f;
      }
      *reinterpret_cast<uint4*>(xs[pl] + r * KC + kk) = pack8_pairs<BITS>(v);
    }
    __syncthreads();
    if (!wave_active) continue;
#pragma unroll
    for (int q = 0; q < NSET; ++q) {
      half2v zl[4], zh[4];
      zero_pairs<BITS>(zraw[q] >> zshift, zoff, zl, zh);
      float4v part[TM][4];
#pragma unroll
      for (int t = 0; t < TM; ++t)
#pragma unroll
        for (int s = 0; s < 4; ++s) part[t][s] = (float4v){0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int st = 0; st < STEPS; ++st) {
        half8v bf[4];
#pragma unroll
        for (int s = 0; s < 4; ++s) bf[s] = b_fragment<BITS>(bw[q][st], s, zl[s], zh[s]);
#pragma unroll
        for (int pl = 0; pl < NA; ++pl)
#pragma unroll
          for (int t = 0; t < TM; ++t) {
            const half8v af = *reinterpret_cast<const half8v*>(xs[pl] + (16 * t + p) * KC + st * 32 + 8 * kb);
#pragma unroll
            for (int s = 0; s < 4; ++s) part[t][s] = __builtin_amdgcn_mfma_f32_16x16x32_f16(af, bf[s], part[t][s], 0, 0, 0);
          }
      }
      float sf[4];
      scales4<ST>(sraw[q], sf);
#pragma unroll
      for (int t = 0; t < TM; ++t)
#pragma unroll
        for (int s = 0; s < 4; ++s)
#pragma unroll
          for (int r = 0; r < 4; ++r) acc[q][t][s][r] = fmaf(sf[s], part[t][s][r], acc[q][t][s][r]);
    }
  }

  if (!colok) return;
#pragma unroll
  for (int t = 0; t < TM; ++t)
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int row = 16 * t + 4 * kb + r;
      if (row >= nrows) continue;
      const size_t slot = (size_t)slot0 + row;
      if constexpr (GATE_UP) {
        __half* hi = static_cast<__half*>(out) + slot * N + ncol;
        __half* lo = hi + out_plane;
#pragma unroll
        for (int s = 0; s < 4; ++s) {
          const float g = acc[0][t][s][r], u = acc[1][t][s][r];
          const float h = g * (1.f / (1.f + expf(-g))) * u;
          const __half hh = __float2half_rn(h);
          hi[s] = hh;
          lo[s] = __float2half_rn(h - __half2float(hh));
        }
      } else {
        float* y = static_cast<float*>(out) + slot * N + ncol;
        const float w = sorted_w[slot];
#pragma unroll
        for (int s = 0; s < 4; ++s) y[s] = acc[0][t][s][r] * w;
      }
    }
}

// out[t][c] = sum over token t's experts, ascending, of y[slot][c] (starting from zero).
__global__ __launch_bounds__(256) void moe_combine_kernel(const float* __restrict__ y, const int* __restrict__ route,
                                                          int T, int E, int k, float* __restrict__ out, int N) {
  const RouteLayout L = route_layout(T, E, k);
  const int* slot_of = route + L.slot_of;
  const int t = blockIdx.y;
  const int c = (blockIdx.x * 256 + threadIdx.x) * 4;
  if (c >= N) return;
  float4 s = make_float4(0.f, 0.f, 0.f, 0.f);
  for (int j = 0; j < k; ++j) {
    const float4 v = *reinterpret_cast<const float4*>(y + (size_t)slot_of[t * k + j] * N + c);
    s.x += v.x; s.y += v.y; s.z += v.z; s.w += v.w;
  }
  *reinterpret_cast<float4*>(out + (size_t)t * N + c) = s;
}

template <int BITS, int KC, bool GATE_UP>
static int launch_moe_gemm(const void* a, const int* route, int T, int E, int k, const int32_t* qw0, const int32_t* qz0,
                           const void* sc0, const int32_t* qw1, const int32_t* qz1, const void* sc1, int sdt, void* out,
                           int K, int N, int gs, float zoff, hipStream_t st) {
  const RouteLayout L = route_layout(T, E, k);
  const int per = 32 / BITS;
  const size_t qws = (size_t)(K / per) * N, qzs = (size_t)(K / gs) * (N / per), scs = (size_t)(K / gs) * N;
  dim3 grid((N + 255) / 256, L.max_tiles);
  // gate_up writes h as two planes of T*k x N halves; down reads them (a_plane = T*k x K)
  const size_t a_plane = GATE_UP ? 0 : (size_t)T * k * K;
  const size_t out_plane = GATE_UP ? (size_t)T * k * N : 0;
  if (sdt == MIQ_F16)
    hipLaunchKernelGGL((moe_gemm_kernel<BITS, KC, GATE_UP, __half>), grid, dim3(256), 0, st,
                       static_cast<const __half*>(a), route, T, E, k, reinterpret_cast<const uint32_t*>(qw0),
                       reinterpret_cast<const uint32_t*>(qz0), static_cast<const __half*>(sc0),
                       reinterpret_cast<const uint32_t*>(qw1), reinterpret_cast<const uint32_t*>(qz1),
                       static_cast<const __half*>(sc1), qws, qzs, scs, a_plane, out, out_plane, K, N, gs, zoff);
  else
    hipLaunchKernelGGL((moe_gemm_kernel<BITS, KC, GATE_UP, float>), grid, dim3(256), 0, st,
                       static_cast<const __half*>(a), route, T, E, k, reinterpret_cast<const uint32_t*>(qw0),
                       reinterpret_cast<const uint32_t*>(qz0), static_cast<const float*>(sc0),
                       reinterpret_cast<const uint32_t*>(qw1), reinterpret_cast<const uint32_t*>(qz1),
                       static_cast<const float*>(sc1), qws, qzs, scs, a_plane, out, out_plane, K, N, gs, zoff);
  return check_launch(GATE_UP ? "moe_gate_up" : "moe_down");
}

template <bool GATE_UP>
static int moe_gemm(const void* a, const int* route, int T, int E, int k, const int32_t* qw0, const int32_t* qz0,
                    const void* sc0, const int32_t* qw1, const int32_t* qz1, const void* sc1, int sdt, void* out, int K,
                    int N, int gs, int bits, float zoff, hipStream_t st) {
  const int kc = gs % 128 == 0 ? 128 : (gs == 64 ? 64 : (gs == 32 ? 32 : 0));
  MIQ_REQUIRE(kc, MIQ_ERR_UNSUPPORTED, "moe: group size %d (32, 64 or a multiple of 128)", gs);
#define MIQ_MOE_CASE(B, C)                                                                                        \
  if (bits == B && kc == C)                                                                                       \
  return launch_moe_gemm<B, C, GATE_UP>(a, route, T, E, k, qw0, qz0, sc0, qw1, qz1, sc1, sdt, out, K, N, gs, zoff, st)
  MIQ_MOE_CASE(4, 128); MIQ_MOE_CASE(4, 64); MIQ_MOE_CASE(4, 32);
  MIQ_MOE_CASE(8, 128); MIQ_MOE_CASE(8, 64); MIQ_MOE_CASE(8, 32);
#undef MIQ_MOE_CASE
  return fail(MIQ_ERR_UNSUPPORTED, "moe: bits=%d", bits);
}

int check_gptq_dims(const char* who, int K, int N, int gs, int bits);

static int moe_check(const char* who, int T, int E, int k) {
  MIQ_REQUIRE(T >= 0 && E > 0 && E <= 1024 && k > 0 && k <= 32 && k <= E, MIQ_ERR_INVALID,
              "%s: T=%d E=%d k=%d (E <= 1024, 0 < k <= min(32, E))", who, T, E, k);
  MIQ_REQUIRE((size_t)T * k <= (size_t)kMoeMaxTK, MIQ_ERR_UNSUPPORTED, "%s: T*k=%lld exceeds %d", who,
              (long long)T * k, kMoeMaxTK);
  return MIQ_OK;
}

}  // namespace miq

using namespace miq;

extern "C" int miq_moe_route_bytes(int T, int E, int k, size_t* bytes) {
  MIQ_REQUIRE(bytes, MIQ_ERR_INVALID, "moe_route_bytes: null output");
  int rc = moe_check("moe_route_bytes", T, E, k);
  if (rc) return rc;
  *bytes = route_layout(T, E, k).words * 4;
  return MIQ_OK;
}

extern "C" int miq_moe_route(const float* logits, int T, int E, int k, int norm_topk, void* route, size_t route_bytes,
                             void* stream) {
  int rc = moe_check("moe_route", T, E, k);
  if (rc || T == 0) return rc;
  MIQ_REQUIRE(logits && route, MIQ_ERR_INVALID, "moe_route: null pointer");
  MIQ_REQUIRE(route_bytes >= route_layout(T, E, k).words * 4 && aligned(route, 16), MIQ_ERR_INVALID,
              "moe_route: route buffer of %zu bytes (16-byte aligned) needed", route_layout(T, E, k).words * 4);
  const size_t lds = (2 * (size_t)T * k + 2 * (size_t)E + 1) * 4;
  hipLaunchKernelGGL(moe_route_kernel, dim3(1), dim3(1024), lds, static_cast<hipStream_t>(stream), logits, T, E, k,
                     norm_topk, static_cast<int*>(route));
  return check_launch("moe_route");
}

extern "C" int miq_moe_gate_up(const void* x, const void* route, int T, int E, int k, const int32_t* qw_gate,
                               const int32_t* qz_gate, const void* sc_gate, const int32_t* qw_up, const int32_t* qz_up,
                               const void* sc_up, int scales_dtype, void* h, int H, int I, int gs, int bits,
                               float zero_offset, void* stream) {
  int rc = moe_check("moe_gate_up", T, E, k);
  if (rc) return rc;
  rc = check_gptq_dims("moe_gate_up", H, I, gs, bits);
  if (rc || T == 0) return rc;
  MIQ_REQUIRE(x && route && qw_gate && qz_gate && sc_gate && qw_up && qz_up && sc_up && h, MIQ_ERR_INVALID,
              "moe_gate_up: null pointer");
  MIQ_REQUIRE(I % 4 == 0 && H % 32 == 0 && aligned(x, 16) && aligned(qw_gate, 16) && aligned(qw_up, 16) && aligned(route, 16),
              MIQ_ERR_ALIGN, "moe_gate_up: alignment (x, weights, route 16 bytes; I %% 4, H %% 32)");
  MIQ_REQUIRE(zero_offset == (float)(int)zero_offset && zero_offset >= 0.f && zero_offset <= 8.f, MIQ_ERR_UNSUPPORTED,
              "moe_gate_up: zero_offset %g", zero_offset);
  return moe_gemm<true>(x, static_cast<const int*>(route), T, E, k, qw_gate, qz_gate, sc_gate, qw_up, qz_up, sc_up,
                        scales_dtype, h, H, I, gs, bits, zero_offset, static_cast<hipStream_t>(stream));
}

extern "C" int miq_moe_down(const void* h, const void* route, int T, int E, int k, const int32_t* qw, const int32_t* qz,
                            const void* sc, int scales_dtype, float* y, int I, int H, int gs, int bits, float zero_offset,
                            void* stream) {
  int rc = moe_check("moe_down", T, E, k);
  if (rc) return rc;
  rc = check_gptq_dims("moe_down", I, H, gs, bits);
  if (rc || T == 0) return rc;
  MIQ_REQUIRE(h && route && qw && qz && sc && y, MIQ_ERR_INVALID, "moe_down: null pointer");
  MIQ_REQUIRE(H % 4 == 0 && I % 32 == 0 && aligned(h, 16) && aligned(qw, 16) && aligned(route, 16), MIQ_ERR_ALIGN,
              "moe_down: alignment (h, weights, route 16 bytes; H %% 4, I %% 32)");
  MIQ_REQUIRE(zero_offset == (float)(int)zero_offset && zero_offset >= 0.f && zero_offset <= 8.f, MIQ_ERR_UNSUPPORTED,
              "moe_down: zero_offset %g", zero_offset);
  return moe_gemm<false>(h, static_cast<const int*>(route), T, E, k, qw, qz, sc, nullptr, nullptr, nullptr,
                         scales_dtype, y, I, H, gs, bits, zero_offset, static_cast<hipStream_t>(stream));
}

extern "C" int miq_moe_combine(const float* y, const void* route, int T, int E, int k, float* out, int H,
                               void* stream) {
  int rc = moe_check("moe_combine", T, E, k);
  if (rc || T == 0) return rc;
  MIQ_REQUIRE(y && route && out, MIQ_ERR_INVALID, "moe_combine: null pointer");
  MIQ_REQUIRE(H % 4 == 0 && aligned(y, 16) && aligned(out, 16), MIQ_ERR_ALIGN, "moe_combine: alignment");
  dim3 grid((H / 4 + 255) / 256, T);
  hipLaunchKernelGGL(moe_combine_kernel, grid, dim3(256), 0, static_cast<hipStream_t>(stream), y,
                     static_cast<const int*>(route), T, E, k, out, H);
  return check_launch("moe_combine");
}
