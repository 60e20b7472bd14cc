// Sparse mixture-of-experts MLP on gfx950: device-side routing, expert-grouped GPTQ GEMMs on the
// matrix cores, and a deterministic combine. No step needs the host, so a decode step with MoE
// layers can be captured in a graph with its routing live.
//
//   route    logits [T][E] fp32 -> float64 softmax -> top-k -> (optional) renormalisation;
//            per token its k experts in ascending order with fp32 weights; per expert the list
//            of its (token, weight) slots in ascending token order ("sorted slots"); and a
//            table of row tiles (expert, first slot, rows) that the GEMMs walk.
//   gate_up  h[slot] = silu(x[token] @ Wg[e]) * (x[token] @ Wu[e])   (fp32)
//   down     y[slot] = w[slot] * (h[slot] @ Wd[e])                    (fp32)
//   combine  out[t] = sum over t's experts in ascending order of y[slot]  (fp32)
//
// The combine order (experts ascending, starting from zero) and the fp32 weight multiply are the
// reference's (`webtorch/lm_engine.py:294-333`). The GEMMs use the prefill GEMM's exact
// dequantization and MFMA mapping (see gptq_gemm.hip); a workgroup takes one row tile of one
// expert (up to kMoeBM rows) and 512 (down) or 128 (gate_up) output columns.
//
// fp32 activations (the intermediate h always; x when the caller's is fp32) go through the fp16
// matrix cores as two fp16 planes of a row scaled by a power of two: v = a * 2^s with s chosen so
// the row's largest |a| is just below 2^15, hi = fp16(v), lo = fp16(v - hi), both multiplied by
// the same weight fragments and the sum scaled back by 2^-s (exact). That keeps about 22
// significant bits relative to the row's largest value with no fp16 range limit. The row scale
// of x comes from a small pass over x; that of h from the maxima the gate_up epilogue takes
// (an atomic max per row and workgroup into a per-slot word the router zeroed). NaN and
// infinite rows keep scale 1, so they propagate.
#include <algorithm>
#include <type_traits>

#include "miq_common.h"
#include "moe_route.h"

namespace miq {

constexpr int kSlotWaves = 16;   // waves of the slot kernel (1024 threads), one chunk of picks each
// waves per grouped-GEMM workgroup (measured: eight down waves sharing a staged h chunk cut
// the down GEMM 44.4 -> 43.2 us at T = 256, H = 2048, 128 experts; eight gate_up waves made it
// slower, 56.8 -> 62.4 us)
constexpr int kMoeWavesGateUp = 4;
constexpr int kMoeWavesDown = 8;

// 2^s with s making m * 2^s just below 2^15 (1 for zero, NaN or infinite m): the row scale of
// the fp16 hi/lo planes. Its inverse is row_unscale(m), also exact.
__device__ __forceinline__ int row_scale_exp(float m) {
  if (!(m > 0.f) || !(m <= 3.4e38f)) return 0;
  int ex;
  frexpf(m, &ex);  // m < 2^ex
  return min(max(15 - ex, -126), 126);  // any finite maximum lands below 2^15; 2^s stays finite
}
__device__ __forceinline__ float row_scale(float m) { return ldexpf(1.f, row_scale_exp(m)); }
__device__ __forceinline__ float row_unscale(float m) { return ldexpf(1.f, -row_scale_exp(m)); }

// fp32 x rows: the largest |x| of each token, stored as the value row_scale reads.
__global__ __launch_bounds__(256) void moe_xmax_kernel(const float* __restrict__ x, int T, int H, int E, int k,
                                                       int* __restrict__ route) {
  const RouteLayout L = route_layout(T, E, k);
  const int t = blockIdx.x * 4 + (threadIdx.x >> 6), lane = threadIdx.x & 63;
  if (t >= T) return;  // whole waves
  float m = 0.f;
  for (int c = lane * 4; c < H; c += 256) {
    const float4 v = *reinterpret_cast<const float4*>(x + (size_t)t * H + c);
    m = fmaxf(m, fmaxf(fmaxf(fabsf(v.x), fabsf(v.y)), fmaxf(fabsf(v.z), fabsf(v.w))));
    // fmaxf drops NaN: carry it explicitly
    if (v.x != v.x || v.y != v.y || v.z != v.z || v.w != v.w) m = __int_as_float(0x7FC00000);
  }
  const bool nan = __ballot(m != m) != 0ull;
  m = wave_max(m != m ? 0.f : m);
  if (lane == 0) reinterpret_cast<float*>(route + L.x_scale)[t] = nan ? __int_as_float(0x7FC00000) : m;
}

// ------------------------------------------------------------------------------------
// Router, two kernels. Top-k: a wave per token (four per workgroup): float64 softmax over the E
// logits (each lane keeps the probabilities of experts lane, lane + 64, ... in registers), k
// rounds of arg-max over them (lowest index on ties; a pick is set to -1 so it cannot win
// again; lane j keeps pick j), renormalisation over the picks, and the picks stored in
// ascending expert order. Slots: one workgroup of 1024 threads with the picks in LDS counts
// each expert's picks (LDS atomics: sums do not depend on order), turns the counts into offsets
// and row tiles (prefix sums over the experts), and then one wave walks the picks in order and
// hands out each expert's slots, so each expert's rows are in ascending token order.
// Float64 (value, expert) steps within each row of 16 lanes by DPP moves (quad_perm [1,0,3,2],
// [2,3,0,1], row_half_mirror, row_mirror), then the four row results by v_readlane. Maximum and
// arg-max (larger value, then smaller expert) are exact in any pairing, so every lane ends with
// the value a butterfly of shuffles would give. All 64 lanes active.
template <int CTRL> __device__ __forceinline__ double dpp_move_f64(double v) {
  const uint64_t u = __builtin_bit_cast(uint64_t, v);
  const uint32_t lo = (uint32_t)__builtin_amdgcn_update_dpp(0, (int)(uint32_t)u, CTRL, 0xF, 0xF, false);
  const uint32_t hi = (uint32_t)__builtin_amdgcn_update_dpp(0, (int)(uint32_t)(u >> 32), CTRL, 0xF, 0xF, false);
  return __builtin_bit_cast(double, ((uint64_t)hi << 32) | lo);
}
__device__ __forceinline__ double lane_at_f64(double v, int l) {
  const uint64_t u = __builtin_bit_cast(uint64_t, v);
  const uint32_t lo = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)u, l);
  const uint32_t hi = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)(u >> 32), l);
  return __builtin_bit_cast(double, ((uint64_t)hi << 32) | lo);
}
__device__ __forceinline__ double wave_max_f64(double v) {
  v = fmax(v, dpp_move_f64<0xB1>(v));
  v = fmax(v, dpp_move_f64<0x4E>(v));
  v = fmax(v, dpp_move_f64<0x141>(v));
  v = fmax(v, dpp_move_f64<0x140>(v));
  return fmax(fmax(lane_at_f64(v, 0), lane_at_f64(v, 16)), fmax(lane_at_f64(v, 32), lane_at_f64(v, 48)));
}
template <int CTRL> __device__ __forceinline__ void pick_step(double& b, int& e) {
  const double ob = dpp_move_f64<CTRL>(b);
  const int oe = __builtin_amdgcn_update_dpp(0, e, CTRL, 0xF, 0xF, false);
  if (ob > b || (ob == b && oe < e)) {
    b = ob;
    e = oe;
  }
}
__device__ __forceinline__ void wave_pick(double& b, int& e) {
  pick_step<0xB1>(b, e);
  pick_step<0x4E>(b, e);
  pick_step<0x141>(b, e);
  pick_step<0x140>(b, e);
  double bb = lane_at_f64(b, 0);
  int be = __builtin_amdgcn_readlane(e, 0);
#pragma unroll
  for (int r = 16; r < 64; r += 16) {
    const double ob = lane_at_f64(b, r);
    const int oe = __builtin_amdgcn_readlane(e, r);
    if (ob > bb || (ob == bb && oe < be)) {
      bb = ob;
      be = oe;
    }
  }
  b = bb;
  e = be;
}

template <int EPL>  // experts per lane: E <= 64 * EPL
__global__ __launch_bounds__(256) void moe_topk_kernel(const float* __restrict__ logits, int T, int E, int k,
                                                       int norm_topk, int* __restrict__ route) {
  const RouteLayout L = route_layout(T, E, k);
  int* topk_e = route + L.topk_e;
  float* topk_w = reinterpret_cast<float*>(route + L.topk_w);
  const int lane = threadIdx.x & 63;
  const int t = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (t >= T) return;  // whole waves
  {
    const float* lt = logits + (size_t)t * E;
    double pv[EPL];
    double mx = -INFINITY;
#pragma unroll
    for (int i = 0; i < EPL; ++i) {
      const int e = lane + 64 * i;
      pv[i] = e < E ? (double)lt[e] : -INFINITY;
      mx = fmax(mx, pv[i]);
    }
    mx = wave_max_f64(mx);
    double sum = 0.0;
#pragma unroll
    for (int i = 0; i < EPL; ++i)
      if (lane + 64 * i < E) {
        pv[i] = exp(pv[i] - mx);
        sum += pv[i];
      }
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) sum += __shfl_xor(sum, o, 64);
    // a NaN probability (NaN logits) ranks below every number but above a taken pick (-1), so
    // such experts are still picked in index order and keep NaN as their weight
    constexpr double kNanRank = -0.5;
#pragma unroll
    for (int i = 0; i < EPL; ++i) {
      const double pr = pv[i] / sum;
      pv[i] = lane + 64 * i < E ? (pr != pr ? kNanRank : pr) : -1.0;
    }
    // lane j keeps pick j (k <= 32), so no per-lane array is indexed at run time
    int my_e = E;
    double my_p = 0.0;
    double psum = 0.0;
    for (int j = 0; j < k; ++j) {
      double best = -1.0;
      int be = E;
#pragma unroll
      for (int i = 0; i < EPL; ++i)
        if (pv[i] > best) {  // ascending e within the lane: the first of equals stays
          best = pv[i];
          be = lane + 64 * i;
        }
      wave_pick(best, be);
#pragma unroll
      for (int i = 0; i < EPL; ++i)
        if (lane + 64 * i == be) pv[i] = -1.0;
      const double bw = best == kNanRank ? __longlong_as_double(0x7FF8000000000000ll) : best;
      if (lane == j) {
        my_e = be;
        my_p = bw;
      }
      psum += bw;
    }
    // ascending expert order: a pick's rank is the number of picks with a smaller expert
    int rank = 0;
    for (int i = 0; i < k; ++i) rank += __builtin_amdgcn_readlane(my_e, i) < my_e;
    if (lane < k) {
      topk_e[t * k + rank] = my_e;
      topk_w[t * k + rank] = (float)(norm_topk ? my_p / psum : my_p);
    }
  }
}

__global__ __launch_bounds__(1024) void moe_slots_kernel(int T, int E, int k, int* __restrict__ route) {
  const RouteLayout L = route_layout(T, E, k);
  const int* topk_e = route + L.topk_e;
  const float* topk_w = reinterpret_cast<const float*>(route + L.topk_w);
  int* slot_of = route + L.slot_of;
  int* sorted_tok = route + L.sorted_tok;
  float* sorted_w = reinterpret_cast<float*>(route + L.sorted_w);
  int* expert_off = route + L.expert_off;
  int* ntiles = route + L.ntiles;
  int4* tiles = reinterpret_cast<int4*>(route + L.tiles);

  extern __shared__ int lds_i[];
  const int TK = T * k;
  int* se = lds_i;                                   // [TK] chosen experts, ascending per token
  float* sw = reinterpret_cast<float*>(lds_i + TK);  // [TK] their weights
  int* cnt = lds_i + 2 * TK;                         // [E + 1] picks per expert
  int* off = cnt + E + 1;                            // [E + 1] first slot per expert
  int* wsum = off + E + 1;                           // [2][16] wave totals of the scans
  int* cw = wsum + 32;                               // [16][E + 1] per wave chunk: picks, then first slots
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  for (int e = threadIdx.x; e <= E; e += blockDim.x) cnt[e] = 0;
  for (int i = threadIdx.x; i < kSlotWaves * (E + 1); i += blockDim.x) cw[i] = 0;
  for (int i = threadIdx.x; i < TK; i += blockDim.x) route[L.slot_max + i] = 0;  // gate_up's row maxima
  for (int i = threadIdx.x; i < TK; i += blockDim.x) {
    se[i] = topk_e[i];
    sw[i] = topk_w[i];
  }
  __syncthreads();
  for (int i = threadIdx.x; i < TK; i += blockDim.x) atomicAdd(&cnt[se[i]], 1);  // sums: order-free
  __syncthreads();
  // expert e's rows and row tiles, exclusive prefix sums over e (one expert per thread,
  // E <= 1024): wave scans, then the wave totals
  int c = 0, ntl = 0;
  if ((int)threadIdx.x < E) {
    c = cnt[threadIdx.x];
    ntl = (c + kMoeBM - 1) / kMoeBM;
  }
  int pc = c, pt = ntl;  // inclusive scans within the wave
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    const int uc = __shfl_up(pc, o, 64), ut = __shfl_up(pt, o, 64);
    if (lane >= o) {
      pc += uc;
      pt += ut;
    }
  }
  if (lane == 63) {
    wsum[wave] = pc;
    wsum[16 + wave] = pt;
  }
  __syncthreads();
  int bc = 0, bt = 0;
  for (int w = 0; w < wave; ++w) {
    bc += wsum[w];
    bt += wsum[16 + w];
  }
  if ((int)threadIdx.x < E) {
    const int e = threadIdx.x, o = bc + pc - c, t0 = bt + pt - ntl;
    off[e] = o;
    expert_off[e] = o;
    for (int i = 0; i < ntl; ++i) tiles[t0 + i] = make_int4(e, o + i * kMoeBM, min(kMoeBM, c - i * kMoeBM), 0);
    if (e == E - 1) {
      off[E] = o + c;
      expert_off[E] = o + c;
      *ntiles = t0 + ntl;
    }
  }
  // the picks in order, in 16 consecutive chunks (one per wave): each chunk's picks per expert,
  // then per expert the chunks' first slots (its offset plus the earlier chunks' picks), so that
  // every wave can walk its chunk at once and the slots come out as one walk in order would give
  const int C = ((TK + kSlotWaves - 1) / kSlotWaves + 63) & ~63;
  const int i0w = wave * C, i1w = min(TK, i0w + C);
  int* runw = cw + wave * (E + 1);
  for (int i = i0w + lane; i < i1w; i += 64) atomicAdd(&runw[se[i]], 1);  // counts: order-free
  __syncthreads();
  for (int e = threadIdx.x; e < E; e += blockDim.x) {
    int base = off[e];
    for (int w = 0; w < kSlotWaves; ++w) {
      const int t = cw[w * (E + 1) + e];
      cw[w * (E + 1) + e] = base;
      base += t;
    }
  }
  __syncthreads();
  // a wave walks its chunk 64 picks at a time: a pick's slot is the chunk's next slot for its
  // expert plus the earlier lanes with the same expert (the lanes that match it, from ballots
  // over the bits of the expert index)
  for (int i0 = i0w; i0 < i1w; i0 += 64) {
    const int i = i0 + lane;
    const bool valid = i < i1w;
    const int e = valid ? se[i] : E;  // E: a sentinel with its own (unused) counter
    uint64_t m = ~0ull;
#pragma unroll
    for (int b = 0; b < 11; ++b) {  // E <= 1024 < 2^11
      const bool bit = (e >> b) & 1;
      const uint64_t bb = __ballot(bit);
      m &= bit ? bb : ~bb;
    }
    const int rank = __popcll(m & ((1ull << lane) - 1));
    const int base = runw[e];
    if (valid) {
      const int sl = base + rank;
      slot_of[i] = sl;
      sorted_tok[sl] = i / k;
      sorted_w[sl] = sw[i];
    }
    if (rank == 0) runw[e] = base + __popcll(m);
  }
}

// ------------------------------------------------------------------------------------
// Grouped GEMM over row tiles. GATE_UP: two weight sets sharing the activations (x rows,
// gathered through the sorted slots), epilogue h = silu(g) * u in fp32 plus each row's max |h|.
// Otherwise (down): one set over h, epilogue y = w[slot] * acc in fp32. XF32: the activations
// are fp32 and are staged as the row-scaled fp16 hi and lo planes (two MFMAs per weight
// fragment); else (gate_up with fp16 x) they are staged as they are. NW waves share each staged
// activation chunk: 64 columns each (gate_up: half the waves gate, half up, 64 columns of each
// per pair), so more waves per workgroup read the activation rows fewer times.
template <int BITS, int KC, bool GATE_UP, bool XF32, typename ST, int NW>
__global__ __launch_bounds__(64 * NW) void moe_gemm_kernel(
    const void* __restrict__ a_in, int* __restrict__ route, int T, int E, int k,
    const uint32_t* __restrict__ qw0, const uint32_t* __restrict__ qz0, const ST* __restrict__ sc0,
    const uint32_t* __restrict__ qw1, const uint32_t* __restrict__ qz1, const ST* __restrict__ sc1,
    size_t qw_stride, size_t qz_stride, size_t sc_stride, const float* __restrict__ b0, const float* __restrict__ b1,
    float* __restrict__ out, int K, int N, int gs, float zoff) {
  constexpr int PER = 32 / BITS;
  constexpr int TM = kMoeBM / 16;
  constexpr int STEPS = KC / 32;
  constexpr int RB = BITS == 4 ? 1 : 2;
  constexpr int NSET = 1;  // weight sets per wave (gate_up: the first NW / 2 waves gate, the rest up)
  constexpr int NT = 64 * NW;
  constexpr int WCOLS = (GATE_UP ? 32 : 64) * NW;  // columns per workgroup
  constexpr int NA = XF32 ? 2 : 1;            // activation planes (hi and lo)
  constexpr int XW = XF32 ? 2 : 1;            // 16-byte words per 8-value piece
  static_assert(GATE_UP || XF32, "the down projection reads fp32 h");
  __shared__ __align__(16) _Float16 xs[2][NA][kMoeBM * KC];  // chunks alternate between two buffers

  const RouteLayout L = route_layout(T, E, k);
  const int tile = blockIdx.y;
  if (tile >= route[L.ntiles]) return;  // uniform: fewer tiles than the grid allows
  const int4 td = reinterpret_cast<const int4*>(route + L.tiles)[tile];
  const int e = td.x, slot0 = td.y, nrows = td.z;
  const int* sorted_tok = route + L.sorted_tok;
  const float* sorted_w = reinterpret_cast<const float*>(route + L.sorted_w);
  // the maxima the row scales come from: x's per token (gate_up), h's per slot (down)
  const float* row_max = reinterpret_cast<const float*>(route + (GATE_UP ? L.x_scale : L.slot_max));
  auto row_id = [&](int row) { return GATE_UP ? sorted_tok[slot0 + row] : slot0 + row; };

  const int lane = threadIdx.x & 63;
  const int wave = uniform(threadIdx.x >> 6);
  const int p = lane & 15, kb = lane >> 4;
  const int cw = GATE_UP ? wave % (NW / 2) : wave, set = GATE_UP ? wave / (NW / 2) : 0;
  const int ncol = blockIdx.x * WCOLS + cw * 64 + 4 * p;
  const bool colok = ncol < N;
  const bool wave_active = blockIdx.x * WCOLS + cw * 64 < N;
  const int NZ = N / PER;
  const int zshift = (ncol % PER) * BITS;
  const uint32_t* qw[1] = {(set ? qw1 : qw0) + e * qw_stride};
  const uint32_t* qz[1] = {(set ? qz1 : qz0) + e * qz_stride};
  const ST* sc[1] = {(set ? sc1 : sc0) + e * sc_stride};

  float4v acc[NSET][TM][4];
#pragma unroll
  for (int q = 0; q < NSET; ++q)
#pragma unroll
    for (int t = 0; t < TM; ++t)
#pragma unroll
      for (int s4 = 0; s4 < 4; ++s4) acc[q][t][s4] = (float4v){0.f, 0.f, 0.f, 0.f};

  // Register triple buffer: while one K chunk is multiplied, the next two chunks' codes,
  // scales, zero points and activation rows are in flight. Loads use addresses clamped into the
  // matrices (columns past N, the chunk after the last), so no branch surrounds them and the
  // compiler's wait counts stay exact; such values are never used.
  constexpr int XCN = kMoeBM * KC / 8;  // 8-value activation pieces per chunk
  // An activation row of a chunk is KC / 8 16-byte pieces; piece c of row r sits in slot
  // c ^ (r % CPR), so that the 16 rows one MFMA operand read touches fall in different banks
  // (unswizzled, rows KC * 2 bytes apart map to the same banks).
  constexpr int CPR = KC / 8;
  constexpr int XCH = (XCN + NT - 1) / NT;  // per thread
  const int ncl = min(ncol, N - 4);
  size_t xsrc[XCH];  // element offset of each piece's row
  int xdst[XCH];     // its LDS offset (row, k) in each plane, -1: none
  bool xz[XCH];      // a row past the tile: zeros
  float xrs[XCH];    // its row scale (fp32 activations)
#pragma unroll
  for (int j = 0; j < XCH; ++j) {
    const int ci = threadIdx.x + NT * j;
    const int cc = min(ci, XCN - 1);
    const int r = cc / (KC / 8), kk = (cc - r * (KC / 8)) * 8;
    const int rr = min(r, nrows - 1);
    const size_t row = (size_t)row_id(rr);
    xsrc[j] = row * K + kk;
    xdst[j] = ci < XCN ? r * KC + (((kk >> 3) ^ (r % CPR)) << 3) : -1;
    xz[j] = r >= nrows;
    xrs[j] = XF32 ? row_scale(row_max[row]) : 1.f;
  }
  struct Chunk {
    uint4 bw[NSET][STEPS][RB];
    uint4 sraw[NSET];
    uint32_t zraw[NSET];
    uint4 xv[XCH][XW];
  };
  auto load_chunk = [&](int kc0, Chunk& c) {
#pragma unroll
    for (int j = 0; j < XCH; ++j)
#pragma unroll
      for (int w = 0; w < XW; ++w)
        c.xv[j][w] = XF32 ? *reinterpret_cast<const uint4*>(static_cast<const float*>(a_in) + xsrc[j] + kc0 + 4 * w)
                          : *reinterpret_cast<const uint4*>(static_cast<const __half*>(a_in) + xsrc[j] + kc0);
#pragma unroll
    for (int q = 0; q < NSET; ++q) {
#pragma unroll
      for (int st = 0; st < STEPS; ++st)
#pragma unroll
        for (int rb = 0; rb < RB; ++rb) {
          const int row = (kc0 + st * 32) / PER + kb * RB + rb;
          c.bw[q][st][rb] = *reinterpret_cast<const uint4*>(qw[q] + (size_t)row * N + ncl);
        }
      const int g = kc0 / gs;
      c.sraw[q] = load_scales4<ST>(sc[q] + (size_t)g * N + ncl);
      c.zraw[q] = qz[q][(size_t)g * NZ + ncl / PER];
    }
  };
  // 8 halves in k order (words (h0,h1) (h2,h3) (h4,h5) (h6,h7)) into the order the code unpack
  // produces (int4: (x0,x4) (x1,x5) (x2,x6) (x3,x7); int8: (x0,x2) (x1,x3) (x4,x6) (x5,x7))
  auto pair_order = [](uint4 w) {
    if constexpr (BITS == 4)
      return make_uint4((w.x & 0xFFFFu) | (w.z << 16), (w.x >> 16) | (w.z & 0xFFFF0000u),
                        (w.y & 0xFFFFu) | (w.w << 16), (w.y >> 16) | (w.w & 0xFFFF0000u));
    else
      return make_uint4((w.x & 0xFFFFu) | (w.y << 16), (w.x >> 16) | (w.y & 0xFFFF0000u),
                        (w.z & 0xFFFFu) | (w.w << 16), (w.z >> 16) | (w.w & 0xFFFF0000u));
  };
  auto stage = [&](const Chunk& c, int b) {
#pragma unroll
    for (int j = 0; j < XCH; ++j) {
      if (xdst[j] < 0) continue;
      if constexpr (XF32) {
        const uint32_t raw[8] = {c.xv[j][0].x, c.xv[j][0].y, c.xv[j][0].z, c.xv[j][0].w,
                                 c.xv[j][1].x, c.xv[j][1].y, c.xv[j][1].z, c.xv[j][1].w};
        uint32_t hi[4], lo[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const float v0 = xz[j] ? 0.f : __uint_as_float(raw[2 * i]) * xrs[j];
          const float v1 = xz[j] ? 0.f : __uint_as_float(raw[2 * i + 1]) * xrs[j];
          const __half h0 = __float2half_rn(v0), h1 = __float2half_rn(v1);
          hi[i] = (uint32_t)__half_as_ushort(h0) | ((uint32_t)__half_as_ushort(h1) << 16);
          lo[i] = (uint32_t)__half_as_ushort(__float2half_rn(v0 - __half2float(h0))) |
                  ((uint32_t)__half_as_ushort(__float2half_rn(v1 - __half2float(h1))) << 16);
        }
        *reinterpret_cast<uint4*>(&xs[b][0][0] + xdst[j]) = pair_order(make_uint4(hi[0], hi[1], hi[2], hi[3]));
        *reinterpret_cast<uint4*>(&xs[b][NA - 1][0] + xdst[j]) = pair_order(make_uint4(lo[0], lo[1], lo[2], lo[3]));
      } else {
        *reinterpret_cast<uint4*>(&xs[b][0][0] + xdst[j]) =
            pair_order(xz[j] ? make_uint4(0u, 0u, 0u, 0u) : c.xv[j][0]);
      }
    }
  };
  auto multiply = [&](const Chunk& c, int b) {
#pragma unroll
    for (int q = 0; q < NSET; ++q) {
      half2v zl[4], zh[4];
      zero_pairs<BITS>(c.zraw[q] >> zshift, zoff, zl, zh);
      float4v part[TM][4];
#pragma unroll
      for (int t = 0; t < TM; ++t)
#pragma unroll
        for (int s4 = 0; s4 < 4; ++s4) part[t][s4] = (float4v){0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int st = 0; st < STEPS; ++st) {
        half8v bf[4];
#pragma unroll
        for (int s4 = 0; s4 < 4; ++s4) bf[s4] = b_fragment<BITS>(c.bw[q][st], s4, zl[s4], zh[s4]);
#pragma unroll
        for (int pl = 0; pl < NA; ++pl)
#pragma unroll
          for (int t = 0; t < TM; ++t) {
            const int row = 16 * t + p;
            const half8v af = *reinterpret_cast<const half8v*>(xs[b][pl] + row * KC + (((st * 4 + kb) ^ (row % CPR)) << 3));
#pragma unroll
            for (int s4 = 0; s4 < 4; ++s4)
              part[t][s4] = __builtin_amdgcn_mfma_f32_16x16x32_f16(af, bf[s4], part[t][s4], 0, 0, 0);
          }
      }
      float sf[4];
      scales4<ST>(c.sraw[q], sf);
#pragma unroll
      for (int t = 0; t < TM; ++t)
#pragma unroll
        for (int s4 = 0; s4 < 4; ++s4)
#pragma unroll
          for (int r = 0; r < 4; ++r) acc[q][t][s4][r] = fmaf(sf[s4], part[t][s4][r], acc[q][t][s4][r]);
    }
  };
  // chunk i is multiplied while chunks i + 1 and i + 2 are in flight (three register sets). It
  // is staged in LDS buffer i % 2, last read by chunk i - 2's multiply, which every wave has
  // finished once it passed chunk i - 1's barrier: one barrier per chunk.
  auto iter = [&](int kc0, Chunk& cur, Chunk& ahead2) {
    const int b = (kc0 / KC) & 1;
    stage(cur, b);
    __syncthreads();
    load_chunk(min(kc0 + 2 * KC, K - KC), ahead2);
    if (wave_active) multiply(cur, b);
  };
  Chunk c0, c1, c2;
  load_chunk(0, c0);
  load_chunk(min(KC, K - KC), c1);
  for (int kc0 = 0; kc0 < K; kc0 += 3 * KC) {
    iter(kc0, c0, c2);
    if (kc0 + KC < K) iter(kc0 + KC, c1, c0);
    if (kc0 + 2 * KC < K) iter(kc0 + 2 * KC, c2, c1);
  }

  if constexpr (GATE_UP) {
    // the up waves hand their sums to the gate waves of the same columns through LDS
    __shared__ float4v ux[NW / 2][TM][4][64];
    if (set == 1)
#pragma unroll
      for (int t = 0; t < TM; ++t)
#pragma unroll
        for (int s4 = 0; s4 < 4; ++s4) ux[cw][t][s4][lane] = acc[0][t][s4];
    __syncthreads();
    if (set == 1 || !wave_active) return;  // wave-uniform
    unsigned* slot_max = reinterpret_cast<unsigned*>(route + L.slot_max);
#pragma unroll
    for (int t = 0; t < TM; ++t)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int row = 16 * t + 4 * kb + r;  // the same in the 16 lanes of a row of D
        const bool live = row < nrows && colok;
        const float un = XF32 ? row_unscale(row_max[row_id(min(row, nrows - 1))]) : 1.f;
        float m = 0.f;
        float hv[4];
#pragma unroll
        for (int s4 = 0; s4 < 4; ++s4) {
          float g = acc[0][t][s4][r] * un, u = ux[cw][t][s4][lane][r] * un;
          if (b0) {  // the experts' fp32 biases, added to each projection's product
            g += colok ? b0[(size_t)e * N + ncol + s4] : 0.f;
            u += colok ? b1[(size_t)e * N + ncol + s4] : 0.f;
          }
          hv[s4] = g * (1.f / (1.f + expf(-g))) * u;
          m = fmaxf(m, fabsf(hv[s4]));  // NaN: the word check below
          if (hv[s4] != hv[s4]) m = __int_as_float(0x7FC00000);
        }
        if (live) *reinterpret_cast<float4*>(out + (size_t)(slot0 + row) * N + ncol) =
            make_float4(hv[0], hv[1], hv[2], hv[3]);
        // the row's max over this wave's 64 columns: the 16 lanes of the row, by DPP moves
        unsigned mb = live ? __float_as_uint(m) : 0u;  // |h| bits: ordered like the values, NaN above all
        mb = max(mb, (unsigned)__builtin_amdgcn_update_dpp(0, (int)mb, 0xB1, 0xF, 0xF, false));
        mb = max(mb, (unsigned)__builtin_amdgcn_update_dpp(0, (int)mb, 0x4E, 0xF, 0xF, false));
        mb = max(mb, (unsigned)__builtin_amdgcn_update_dpp(0, (int)mb, 0x141, 0xF, 0xF, false));
        mb = max(mb, (unsigned)__builtin_amdgcn_update_dpp(0, (int)mb, 0x140, 0xF, 0xF, false));
        if (p == 0 && row < nrows) atomicMax(slot_max + slot0 + row, mb);
      }
  } else {
    if (!colok) return;
#pragma unroll
    for (int t = 0; t < TM; ++t)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int row = 16 * t + 4 * kb + r;
        if (row >= nrows) continue;
        const size_t slot = (size_t)slot0 + row;
        float* y = out + slot * N + ncol;
        if (b0) {  // (h @ Wd + bias) * w, as the expert's linear then the routing weight
          const float un = row_unscale(row_max[slot]), w = sorted_w[slot];
#pragma unroll
          for (int s4 = 0; s4 < 4; ++s4) y[s4] = (acc[0][t][s4][r] * un + b0[(size_t)e * N + ncol + s4]) * w;
        } else {
          const float wsc = sorted_w[slot] * row_unscale(row_max[slot]);
#pragma unroll
          for (int s4 = 0; s4 < 4; ++s4) y[s4] = acc[0][t][s4][r] * wsc;
        }
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

template <int BITS, int KC, bool GATE_UP, bool XF32>
static int launch_moe_gemm(const void* a, int* route, int T, int E, int k, const int32_t* qw0, const int32_t* qz0,
                           const void* sc0, const int32_t* qw1, const int32_t* qz1, const void* sc1, int sdt,
                           const float* b0, const float* b1, float* out, int K, int N, int gs, float zoff,
                           hipStream_t st) {
  const RouteLayout L = route_layout(T, E, k);
  const int per = 32 / BITS;
  const size_t qws = (size_t)(K / per) * N, qzs = (size_t)(K / gs) * (N / per), scs = (size_t)(K / gs) * N;
  constexpr int NW = GATE_UP ? kMoeWavesGateUp : kMoeWavesDown;
  constexpr int WCOLS = (GATE_UP ? 32 : 64) * NW;
  dim3 grid((N + WCOLS - 1) / WCOLS, L.max_tiles);
  const uint32_t *w0 = reinterpret_cast<const uint32_t*>(qw0), *z0 = reinterpret_cast<const uint32_t*>(qz0);
  const uint32_t *w1 = reinterpret_cast<const uint32_t*>(qw1), *z1 = reinterpret_cast<const uint32_t*>(qz1);
  if (sdt == MIQ_F16)
    hipLaunchKernelGGL((moe_gemm_kernel<BITS, KC, GATE_UP, XF32, __half, NW>), grid, dim3(64 * NW), 0, st, a, route, T, E, k,
                       w0, z0, static_cast<const __half*>(sc0), w1, z1, static_cast<const __half*>(sc1), qws, qzs,
                       scs, b0, b1, out, K, N, gs, zoff);
  else
    hipLaunchKernelGGL((moe_gemm_kernel<BITS, KC, GATE_UP, XF32, float, NW>), grid, dim3(64 * NW), 0, st, a, route, T, E, k,
                       w0, z0, static_cast<const float*>(sc0), w1, z1, static_cast<const float*>(sc1), qws, qzs, scs,
                       b0, b1, out, K, N, gs, zoff);
  return check_launch(GATE_UP ? "moe_gate_up" : "moe_down");
}

template <bool GATE_UP, bool XF32>
static int moe_gemm(const void* a, int* route, int T, int E, int k, const int32_t* qw0, const int32_t* qz0,
                    const void* sc0, const int32_t* qw1, const int32_t* qz1, const void* sc1, int sdt, const float* b0,
                    const float* b1, float* out, int K, int N, int gs, int bits, float zoff, hipStream_t st) {
  const int kc = gs % 128 == 0 ? 128 : (gs == 64 ? 64 : (gs == 32 ? 32 : 0));
  MIQ_REQUIRE(kc, MIQ_ERR_UNSUPPORTED, "moe: group size %d (32, 64 or a multiple of 128)", gs);
#define MIQ_MOE_CASE(B, C)                                                                                        \
  if (bits == B && kc == C)                                                                                       \
  return launch_moe_gemm<B, C, GATE_UP, XF32>(a, route, T, E, k, qw0, qz0, sc0, qw1, qz1, sc1, sdt, b0, b1, out, K, \
                                              N, gs, zoff, st)
  MIQ_MOE_CASE(4, 128); MIQ_MOE_CASE(4, 64); MIQ_MOE_CASE(4, 32);
  MIQ_MOE_CASE(8, 128); MIQ_MOE_CASE(8, 64); MIQ_MOE_CASE(8, 32);
#undef MIQ_MOE_CASE
  return fail(MIQ_ERR_UNSUPPORTED, "moe: bits=%d", bits);
}

// out[t][c] += ys[t][c] * sigmoid(gl[t]) (gl null: += ys), the shared expert's contribution
// (`webtorch/lm_engine.py:322-328`: g = 1 / (1 + exp(-gl)) in fp32, ys * g, out + ys).
__global__ __launch_bounds__(256) void moe_shared_add_kernel(float* __restrict__ out, const float* __restrict__ ys,
                                                             const float* __restrict__ gl, int H) {
  const int t = blockIdx.y;
  const int c = blockIdx.x * 256 + threadIdx.x;
  if (c >= H) return;
  float y = ys[(size_t)t * H + c];
  if (gl) y = y * (1.f / (1.f + expf(-gl[t])));
  out[(size_t)t * H + c] += y;
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
  const hipStream_t st = static_cast<hipStream_t>(stream);
  int* r = static_cast<int*>(route);
  const dim3 g((T + 3) / 4);
  if (E <= 64) hipLaunchKernelGGL(moe_topk_kernel<1>, g, dim3(256), 0, st, logits, T, E, k, norm_topk, r);
  else if (E <= 128) hipLaunchKernelGGL(moe_topk_kernel<2>, g, dim3(256), 0, st, logits, T, E, k, norm_topk, r);
  else if (E <= 256) hipLaunchKernelGGL(moe_topk_kernel<4>, g, dim3(256), 0, st, logits, T, E, k, norm_topk, r);
  else if (E <= 512) hipLaunchKernelGGL(moe_topk_kernel<8>, g, dim3(256), 0, st, logits, T, E, k, norm_topk, r);
  else hipLaunchKernelGGL(moe_topk_kernel<16>, g, dim3(256), 0, st, logits, T, E, k, norm_topk, r);
  // se, sw [T*k]; cnt, off [E+1]; wave sums [32]; per chunk counters [16][E+1]
  const size_t lds = (2 * (size_t)T * k + (2 + kSlotWaves) * ((size_t)E + 1) + 32) * 4;
  if (lds > 64 * 1024 && (rc = require_lds("moe_route", lds))) return rc;
  hipLaunchKernelGGL(moe_slots_kernel, dim3(1), dim3(1024), lds, st, T, E, k, r);
  return check_launch("moe_route");
}

extern "C" int miq_moe_gate_up(const void* x, int x_dtype, void* route, int T, int E, int k, const int32_t* qw_gate,
                               const int32_t* qz_gate, const void* sc_gate, const int32_t* qw_up, const int32_t* qz_up,
                               const void* sc_up, int scales_dtype, const float* bias_gate, const float* bias_up,
                               float* h, int H, int I, int gs, int bits, float zero_offset, void* stream) {
  int rc = moe_check("moe_gate_up", T, E, k);
  if (rc) return rc;
  rc = check_gptq_dims("moe_gate_up", H, I, gs, bits);
  if (rc || T == 0) return rc;
  MIQ_REQUIRE(x && route && qw_gate && qz_gate && sc_gate && qw_up && qz_up && sc_up && h, MIQ_ERR_INVALID,
              "moe_gate_up: null pointer");
  MIQ_REQUIRE(x_dtype == MIQ_F16 || x_dtype == MIQ_F32, MIQ_ERR_UNSUPPORTED, "moe_gate_up: x dtype");
  MIQ_REQUIRE(I % 4 == 0 && H % 32 == 0 && aligned(x, 16) && aligned(h, 16) && aligned(qw_gate, 16) &&
                  aligned(qw_up, 16) && aligned(route, 16),
              MIQ_ERR_ALIGN, "moe_gate_up: alignment (x, h, weights, route 16 bytes; I %% 4, H %% 32)");
  MIQ_REQUIRE(zero_offset == (float)(int)zero_offset && zero_offset >= 0.f && zero_offset <= 8.f, MIQ_ERR_UNSUPPORTED,
              "moe_gate_up: zero_offset %g", zero_offset);
  MIQ_REQUIRE(!bias_gate == !bias_up, MIQ_ERR_INVALID, "moe_gate_up: give both expert biases or neither");
  const hipStream_t st = static_cast<hipStream_t>(stream);
  int* r = static_cast<int*>(route);
  if (x_dtype == MIQ_F32) {
    hipLaunchKernelGGL(moe_xmax_kernel, dim3((T + 3) / 4), dim3(256), 0, st, static_cast<const float*>(x), T, H, E, k, r);
    rc = check_launch("moe_gate_up row scales");
    if (rc) return rc;
    return moe_gemm<true, true>(x, r, T, E, k, qw_gate, qz_gate, sc_gate, qw_up, qz_up, sc_up, scales_dtype, bias_gate,
                                bias_up, h, H, I, gs, bits, zero_offset, st);
  }
  return moe_gemm<true, false>(x, r, T, E, k, qw_gate, qz_gate, sc_gate, qw_up, qz_up, sc_up, scales_dtype, bias_gate,
                               bias_up, h, H, I, gs, bits, zero_offset, st);
}

extern "C" int miq_moe_down(const float* h, void* route, int T, int E, int k, const int32_t* qw, const int32_t* qz,
                            const void* sc, int scales_dtype, const float* bias, float* y, int I, int H, int gs, int bits,
                            float zero_offset, void* stream) {
  int rc = moe_check("moe_down", T, E, k);
  if (rc) return rc;
  rc = check_gptq_dims("moe_down", I, H, gs, bits);
  if (rc || T == 0) return rc;
  MIQ_REQUIRE(h && route && qw && qz && sc && y, MIQ_ERR_INVALID, "moe_down: null pointer");
  MIQ_REQUIRE(H % 4 == 0 && I % 32 == 0 && aligned(h, 16) && aligned(qw, 16) && aligned(route, 16), MIQ_ERR_ALIGN,
              "moe_down: alignment (h, weights, route 16 bytes; H %% 4, I %% 32)");
  MIQ_REQUIRE(zero_offset == (float)(int)zero_offset && zero_offset >= 0.f && zero_offset <= 8.f, MIQ_ERR_UNSUPPORTED,
              "moe_down: zero_offset %g", zero_offset);
  return moe_gemm<false, true>(h, static_cast<int*>(route), T, E, k, qw, qz, sc, nullptr, nullptr, nullptr,
                               scales_dtype, bias, nullptr, y, I, H, gs, bits, zero_offset,
                               static_cast<hipStream_t>(stream));
}

extern "C" int miq_moe_shared_add(float* out, const float* ys, const float* gate_logits, int T, int H, void* stream) {
  MIQ_REQUIRE(T >= 0 && H > 0, MIQ_ERR_INVALID, "moe_shared_add: T=%d H=%d", T, H);
  if (T == 0) return MIQ_OK;
  MIQ_REQUIRE(out && ys, MIQ_ERR_INVALID, "moe_shared_add: null pointer");
  hipLaunchKernelGGL(moe_shared_add_kernel, dim3((H + 255) / 256, T), dim3(256), 0, static_cast<hipStream_t>(stream),
                     out, ys, gate_logits, H);
  return check_launch("moe_shared_add");
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
