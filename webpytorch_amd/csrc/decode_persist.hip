// Persistent decode step for gfx950: one launch per token for a Qwen2-style int4 GPTQ decoder
// (the captured one-token step of `webtorch/llm.py:1591-1616`), with no grid-wide barrier.
//
// Every workgroup (1024 threads, one per CU) has a role for all layers:
//   * a 64-column tile of the q|k|v projection;
//   * a query head: RoPE and attention over the cache, publishing the head's 64 outputs;
//   * a 64-column tile of the o projection over all heads' outputs, plus the residual:
//     hmid(l) = h(l) + att @ Wo;
//   * a 64-column tile of the gate|up projection (32 gate and the matching 32 up columns, whose
//     silu(gate) * up it publishes);
//   * a (64-column tile, K-slice) of the down projection.
// A layer is five dependent hops: h(l) -> q|k|v -> heads -> o tiles (hmid) -> gate|up -> down ->
// h(l + 1).
//
// Single-writer results (q|k|v, the heads' outputs, hmid, gate|up) are (tag << 32) | fp32 bits
// words written and read at device scope (they bypass the per-XCD L2); a tag names (token,
// layer, phase) and never repeats between consecutive tokens, so no reset is needed.
// h(l + 1) = hmid(l) + the down projection's K-slices is summed in fixed point instead: each
// K-slice, and the gate|up tiles for the residual hmid(l), add their term to a 64-bit word per
// (layer, column) as round(p 2^24) + 2^46 with 1 in a count field, by one device-scope atomic,
// and a consumer polls the words until the count is complete (one word per column instead of one
// per K-slice and column). Integer sums do not depend on the order of arrival, so a step is
// deterministic; a term the fixed point cannot hold (NaN, Inf, |p| >= 2^22) takes the exact
// escape of mma_tile.h (an fp32 side slot read back in term order). The words of a token sit in
// one of two banks (by the parity of the token's epoch); each step zeroes the other bank for the
// next step, and the kernel boundary orders the two. (Terms that many workgroups add to the same
// words serialize at the coherence point, so the o projection is a hop of its own: the heads
// publish their 64 outputs each and every o tile reads all of them, NH * 64 words, where heads
// publishing their shares of the o projection (H words each, summed by the tiles) made a
// 2.6 us hop against 0.9 us for the q|k|v -> heads one.)
// A role's weights for layer l are issued as soon as its layer l-1 work is done, a whole layer
// ahead of their use, so the HBM traffic of the weights overlaps the chain of dependent steps.
//
// After the last layer every workgroup takes 64-column tiles of the tied head, keeps a running
// arg-max, and publishes it; workgroup 0 combines the partials in workgroup order, writes the
// token id, appends it to the history and advances the position, exactly as argmax_kernel does.
//
// Waits are bounded: a workgroup that is still waiting `spin_limit` wall-clock ticks after it
// started sets an error bit and leaves, so every wait chain ends and the grid drains. A step that
// failed leaves its exchange words and bank dirty: later steps see the bit and leave at entry,
// and the host resets the workspace and runs the rest of the sequence as the launch sequence.
// All workgroups must be resident at once; the host sizes the grid to the CU count and checks
// occupancy, and the step must not share the GPU with other work.
//
// Control words at the start of the workspace (uint32): [0] epoch of the last token done,
// [1] error bits (1: wait timed out, 2: position past the cache).
#include <math.h>

#include <stdlib.h>

#include <algorithm>

#include "miq_common.h"
#include "mma_tile.h"

// The elementwise steps (RMSNorm, RoPE, SiLU, softmax) round every product and sum separately,
// as the reference's numpy expressions do; explicit fmaf() calls are unaffected.
#pragma clang fp contract(off)

namespace miq {
namespace pd {

using namespace mt;

constexpr int kThreads = 1024, kWaves = 16, kTile = 64, kMaxSPQ = 8, kSlots = 20;
enum Slot { QKV_QW, QKV_QZ, QKV_SC, QKV_B, O_QW, O_QZ, O_SC, GU_QW, GU_QZ, GU_SC, D_QW, D_QZ, D_SC, IN_LN, POST_LN, KC, VC };
enum Phase { P_QKV = 0, P_ATT = 1, P_HMID = 2, P_GU = 3, P_AMAX = 5 };

struct Params {
  const uint64_t* layers;  // [L][kSlots] device addresses, indexed by Slot
  const __half* embed;
  const uint32_t* head_qw;
  const uint32_t* head_qz;
  const float* head_sc;
  const float* final_norm;
  const float* cos_t;
  const float* sin_t;
  int32_t* ids;
  int32_t* history;
  int32_t* state;
  float* logits;
  uint32_t* ctl;
  uint64_t *tq, *tatt, *thmid, *tgu, *tamax;  // q|k|v, heads' outputs [NH][64], hmid, silu(gate) * up, arg-max
  unsigned long long* fx;  // bank 0 of the fixed-point words of h(l + 1) (bank 1 at fx + bank_words)
  float* fside;            // escape slots: term s of word i at fside + s * LH + i
  size_t bank_words;       // 64-bit words per bank: LH sums, then LH 32-bit masks
  int L, H, NH, NKV, I, V, LMAX, gs, lgs, hist_len, ksd;  // lgs = log2(gs)
  int nq, na, no, ngu, nd;  // workgroups per role (nd = no * ksd, no = H / 64)
  int lds_a, lds_x;      // LDS regions (floats): exchange/staging, activations
  float eps, scale, zoff, head_zoff;
  long long spin_limit;
  unsigned long long* trace;  // null, or [G][L + 2][8] wall-clock stamps of the phase marks below
};

// Phase mark k of layer l of this workgroup: in the kernel instantiated with TR (the one
// miq_decode_persistent_trace launches) thread 0 stores the wall clock; otherwise nothing (a
// runtime test of the trace pointer at every mark cost 1.7% of the step).
#define PD_MARK(l, k)                                                                                \
  do {                                                                                               \
    if constexpr (TR)                                                                                \
      if (threadIdx.x == 0) p.trace[((size_t)blockIdx.x * (p.L + 2) + (l)) * 8 + (k)] = wall_clock64(); \
  } while (0)

__device__ __forceinline__ void tput(uint64_t* p, uint32_t tag, float v) {
  __hip_atomic_store(p, ((uint64_t)tag << 32) | __float_as_uint(v), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ uint64_t tget(const uint64_t* p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

struct Ctx {
  long long deadline;
  uint32_t ep;
  int L;
  __device__ uint32_t tag(int l, int ph) const { return ep * (uint32_t)(8 * (L + 1)) + 8u * (uint32_t)l + (uint32_t)ph; }
};

// Columns c0.. of h(l + 1) as fixed-point words of this token's bank, with their masks and
// escape slots.
struct Fx {
  unsigned long long* w;
  uint32_t* m;
  float* side;
  size_t stride;
};
__device__ __forceinline__ Fx fx_row(const Params& p, uint32_t ep, int l, int c0 = 0) {
  const size_t n = (size_t)p.L * p.H, off = (size_t)l * p.H + c0;
  unsigned long long* bank = p.fx + (ep & 1u) * p.bank_words;
  return {bank + off, reinterpret_cast<uint32_t*>(bank + n) + off, p.fside + off, n};
}
// Term `term` adds v to column i (no return value is waited for).
__device__ __forceinline__ void fx_put(const Fx& r, int i, float v, int term) {
  const FixEsc e{r.m + i, r.side + i, r.stride};
  (void)fix_issue(r.w + i, fix_word(v), v, e, term);
}
// The value of a complete word of `terms` terms (escaped terms added in term order).
__device__ __forceinline__ float fx_value(unsigned long long w, int terms, const Fx& r, int i) {
  const long long v = (long long)(w & ((1ull << kFixEscShift) - 1)) - (long long)terms * (long long)kFixBias;
  float s = (float)v * (1.f / kFixScale);
  if ((w >> kFixEscShift) & 63ull) {
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
    const uint32_t m = __hip_atomic_load(r.m + i, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    for (int t = 0; t < terms; ++t)
      if ((m >> t) & 1u) s += __hip_atomic_load(r.side + (size_t)t * r.stride + i, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
  return s;
}

// After a wave's polling: true (uniformly) unless a wave passed the deadline. late is
// wave-uniform (a vote and the scalar clock decide it): one flag per wave and one barrier
// (__syncthreads_or costs three). Every wait is followed by at least one more barrier before
// the next wait writes the flags, so no wave rewrites a flag while another still reads it.
__device__ __forceinline__ bool all_on_time(bool late, int* flags) {
  if ((threadIdx.x & 63) == 0) flags[threadIdx.x >> 6] = late ? 1 : 0;
  __syncthreads();
  const int4* f = reinterpret_cast<const int4*>(flags);
  int any = 0;
#pragma unroll
  for (int q = 0; q < kWaves / 4; ++q) {
    const int4 t = f[q];
    any |= t.x | t.y | t.z | t.w;
  }
  return any == 0;
}

// Polls n tagged words (word i at base + off(i)) until word i carries tagf(i), leaving their values
// in dst[0..n) (LDS). Called by the whole workgroup with the same arguments; n <= NPL * 1024.
// Each wave polls its own words until they are all current (no barrier per round), then the
// workgroup meets once. Returns false (uniformly) once a wave has passed the deadline.
template <int NPL, typename F, typename T>
__device__ bool wait_tagged(int n, const Ctx& c, const uint64_t* base, F off, T tagf, float* dst, int* flags) {
  const int tid = opaque_tid();
  bool late = false;
  for (;;) {
    uint64_t v[NPL];
#pragma unroll
    for (int j = 0; j < NPL; ++j)
      if (j * kThreads < n) v[j] = tget(base + (uint32_t)off(min(tid + j * kThreads, n - 1)));
    bool ok = true;
#pragma unroll
    for (int j = 0; j < NPL; ++j) {
      const int i = tid + j * kThreads;
      if (j * kThreads < n && i < n) {
        ok &= (uint32_t)(v[j] >> 32) == tagf(i);
        dst[i] = __uint_as_float((uint32_t)v[j]);
      }
    }
    if (__all(ok)) break;
    if (wall_clock64() > c.deadline) {  // wave-uniform (scalar clock)
      late = true;
      break;
    }
    __builtin_amdgcn_s_sleep(1);
  }
  return all_on_time(late, flags);
}

// Polls the n fixed-point words of row r until each holds `terms` terms, leaving their values in
// dst[0..n) (LDS); n <= NPL * 1024. Same contract as wait_tagged.
template <int NPL>
__device__ bool wait_fixed(int n, const Ctx& c, const Fx& r, int terms, float* dst, int* flags) {
  const int tid = opaque_tid();
  bool late = false;
  unsigned long long v[NPL];
  for (;;) {
#pragma unroll
    for (int j = 0; j < NPL; ++j)
      if (j * kThreads < n)
        v[j] = __hip_atomic_load(r.w + min(tid + j * kThreads, n - 1), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    bool ok = true;
#pragma unroll
    for (int j = 0; j < NPL; ++j)
      if (j * kThreads < n && tid + j * kThreads < n) ok &= (int)(v[j] >> kFixCountShift) == terms;
    if (__all(ok)) break;
    if (wall_clock64() > c.deadline) {
      late = true;
      break;
    }
    __builtin_amdgcn_s_sleep(1);
  }
  if (!late) {
#pragma unroll
    for (int j = 0; j < NPL; ++j) {
      const int i = tid + j * kThreads;
      if (j * kThreads < n && i < n) dst[i] = fx_value(v[j], terms, r, i);
    }
  }
  return all_on_time(late, flags);
}

// RMSNorm applied after the projection, which is linear: RMSNorm(h) @ W = ((h * w) @ W) / r with
// r = sqrt(mean(h^2) + eps) one scalar per token, so the block reduction for r overlaps the
// matrix work instead of preceding it. norm_stage scales this thread's chunk by the norm weight
// and leaves the wave's sum of squares in red16[wave] (visible after the next barrier);
// norm_r combines them in wave order.
__device__ __forceinline__ void norm_stage(float* v, const float4* w, float* red16) {
  float ss = 0.f;
#pragma unroll
  for (int j = 0; j < 8; ++j) ss = ss + v[j] * v[j];
  ss = wave_sum(ss);
  if ((threadIdx.x & 63) == 0) red16[threadIdx.x >> 6] = ss;
  v[0] = v[0] * w[0].x;
  v[1] = v[1] * w[0].y;
  v[2] = v[2] * w[0].z;
  v[3] = v[3] * w[0].w;
  v[4] = v[4] * w[1].x;
  v[5] = v[5] * w[1].y;
  v[6] = v[6] * w[1].z;
  v[7] = v[7] * w[1].w;
}
__device__ __forceinline__ float norm_r(const float* red16, int H, float eps) {
  float t = 0.f;
#pragma unroll
  for (int w = 0; w < kWaves; ++w) t += red16[w];
  return sqrtf(t / (float)H + eps);
}

// This thread's chunk (8 values) of an RMSNorm weight vector of H values, loaded ahead.
__device__ __forceinline__ void norm_prefetch(float4* w, const float* nw, int H) {
  const int ch = min((int)threadIdx.x, H / 8 - 1);
  w[0] = ldgf4(nw + ch * 8);
  w[1] = ldgf4(nw + ch * 8 + 4);
  pin(w[0]);
  pin(w[1]);
}

__device__ __forceinline__ float rope1(const float* row, int d, int half, float c, float s) {
  const float rv = d < half ? -row[d + half] : row[d - half];
  return row[d] * c + rv * s;
}

__device__ __forceinline__ bool better(float v, int i, float bv, int bi) {
  return v > bv || (v == bv && i < bi);
}
// (value, index) arg-max over a wave with all 64 lanes active, NaN losing to any number: DPP
// moves within each row of 16, then the four row winners by v_readlane. The order (larger value,
// then smaller index) is total, so every lane ends with the same winner whatever the pairing.
template <int CTRL> __device__ __forceinline__ void amax_step(float& v, int& i) {
  const float ov = dpp_move<CTRL>(v);
  const int oi = __builtin_amdgcn_update_dpp(0, i, CTRL, 0xF, 0xF, false);
  if (better(ov, oi, v, i) || (v != v && ov == ov)) {
    v = ov;
    i = oi;
  }
}
__device__ __forceinline__ void wave_argmax(float& v, int& i) {
  amax_step<0xB1>(v, i);
  amax_step<0x4E>(v, i);
  amax_step<0x141>(v, i);
  amax_step<0x140>(v, i);
  float bv = lane_at(v, 0);
  int bi = __builtin_amdgcn_readlane(i, 0);
#pragma unroll
  for (int r = 16; r < 64; r += 16) {
    const float ov = lane_at(v, r);
    const int oi = __builtin_amdgcn_readlane(i, r);
    if (better(ov, oi, bv, bi) || (bv != bv && ov == ov)) {
      bv = ov;
      bi = oi;
    }
  }
  v = bv;
  i = bi;
}

// LDS carve-up: hin (exchange words and scratch), xs (fp32 activations), xa (A operand steps),
// cx (bias and x sums per step), red (16 k-parts x 64 columns), red16 (wave scalars), qkv
// (rotated q, k and the new v), flags (wait votes).
struct Lds {
  float *hin, *xs;
  unsigned char* xa;
  float2* cx;
  float *red, *red16, *qkv;
  int* flags;  // two sets of wait votes
};
constexpr int kQkvFloats = 192;

#define MIQ_PD_INLINE __device__ __attribute__((always_inline)) inline

// h(l) for this thread's 8-value chunk (threads < H / 8; the others get zeros), also left in
// raw[0..H): layer 0 is the current token's embedding row (each thread writes its own chunk of
// raw); later layers wait for the fixed-point words of h(l) (the down projection's K-slices plus
// hmid(l - 1)).
MIQ_PD_INLINE bool gather_h(const Params& p, const Ctx& c, const Lds& s, int l, int tok, float* raw, float* v) {
  const int H = p.H, ch = threadIdx.x;
  if (l > 0 && !wait_fixed<1>(H, c, fx_row(p, c.ep, l - 1), p.ksd + 1, raw, s.flags)) return false;
#pragma unroll
  for (int j = 0; j < 8; ++j) v[j] = 0.f;
  if (ch < H / 8) {
    if (l == 0) {
      if (tok >= 0 && tok < p.V) {
        const __half* e = p.embed + (size_t)tok * H + ch * 8;
#pragma unroll
        for (int j = 0; j < 8; ++j) v[j] = __half2float(e[j]);
      }
#pragma unroll
      for (int j = 0; j < 8; ++j) raw[ch * 8 + j] = v[j];  // the thread's own chunk, as the wait leaves it
    } else {
#pragma unroll
      for (int j = 0; j < 8; ++j) v[j] = raw[ch * 8 + j];
    }
  }
  return true;
}

// q|k|v projection, columns [64 t, 64 t + 64): RMSNorm(h(l)) @ Wqkv + bias.
template <int SA, bool TR>
MIQ_PD_INLINE bool role_qkv(const Params& p, const Ctx& c, const Lds& s, int t, int tok) {
  float zo = p.zoff;
  pin(zo);
  const int H = p.H, NQ = (p.NH + 2 * p.NKV) * 64, c0 = t * kTile;
  for (int l = 0; l < p.L; ++l) {
    const uint64_t* lt = p.layers + (size_t)l * kSlots;
    Tile<__half, SA> w;
    tile_issue<__half, SA, true, true>(w, (const uint32_t*)lt[QKV_QW], (const uint32_t*)lt[QKV_QZ], (const __half*)lt[QKV_SC], NQ, c0, 0,
               H / 32, p.lgs);
    float4 nw[2];
    norm_prefetch(nw, (const float*)lt[IN_LN], H);
    const float* bias = (const float*)lt[QKV_B];
    float bv = (bias && threadIdx.x < 64) ? ldg(bias + min(c0 + (int)threadIdx.x, NQ - 1)) : 0.f;
    pin(bv);
    PD_MARK(l, 0);
    float v[8];
    if (!gather_h(p, c, s, l, tok, s.hin, v)) return false;
    PD_MARK(l, 1);
    const int ch = threadIdx.x;
    norm_stage(v, nw, s.red16);
    if (ch < H / 8) stage_digits(ch, v, s.xa, s.cx);
    __syncthreads();
    PD_MARK(l, 3);
    const float4 acc = tile_mma_i8(w, s.xa, s.cx, 0, c0, p.lgs, zo);
    PD_MARK(l, 5);
    float y = tile_sum(acc, s.red);
    PD_MARK(l, 4);
    if (threadIdx.x < 64 && c0 + (int)threadIdx.x < NQ) {
      y = y / norm_r(s.red16, H, p.eps);
      if (bias) y += bv;
      tput(p.tq + c0 + threadIdx.x, c.tag(l, P_QKV), y);
    }
    PD_MARK(l, 2);
    __syncthreads();
  }
  return true;
}

// q . k over 16 dimensions (q from LDS, k in registers), fused multiply-adds in order.
__device__ __forceinline__ float dot16(const float* q, const float4* k) {
  float a = 0.f;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    a = fmaf(q[4 * i], k[i].x, a);
    a = fmaf(q[4 * i + 1], k[i].y, a);
    a = fmaf(q[4 * i + 2], k[i].z, a);
    a = fmaf(q[4 * i + 3], k[i].w, a);
  }
  return a;
}

// Query head hq at position pos over positions 0..pos, all layers: RoPE of q and of the kv
// head's new k (the first query head of each group writes k and v into the caches), scores
// (q . k) * scale, softmax, sum p v, published as the head's 64 tagged outputs. Each wave takes
// every 16th position (four threads per position for the scores, a lane per dimension for the
// weighted sum) with a softmax of its own (running maximum and sum), and the 16 waves' partials
// are combined once, rescaled to the common maximum: no barrier between the scores, the softmax
// and the weighted sum. The cache rows of the first 256 positions and the
// RoPE row are loaded before q/k/v are waited for.
template <bool TR>
MIQ_PD_INLINE bool role_attn(const Params& p, const Ctx& c, const Lds& s, int hq, int pos) {
  const int NH = p.NH, NKV = p.NKV, LMAX = p.LMAX, rep = NH / NKV, g = hq / rep, S = pos + 1;
  float* qs = s.qkv;
  float* kn = s.qkv + 64;
  float* vn = s.qkv + 128;
  const int jr = (threadIdx.x & 63) < 32 ? (threadIdx.x & 63) : (threadIdx.x & 63) - 32;
  const float cs = p.cos_t[(size_t)pos * 32 + jr], sn = p.sin_t[(size_t)pos * 32 + jr];
  for (int l = 0; l < p.L; ++l) {
    // thread indices recomputed per layer (opaque_tid): address math hoisted out of the layer
    // loop would hold registers for the whole token
    const int tid = opaque_tid(), wave = uniform(tid >> 6), lane = tid & 63, qq = tid & 3;
    const int jq = wave + 16 * (lane >> 2);  // this quad's position in a 256-position chunk
    const uint64_t* lt = p.layers + (size_t)l * kSlots;
    float* kc = (float*)lt[KC] + (size_t)g * LMAX * 64;
    float* vc = (float*)lt[VC] + (size_t)g * LMAX * 64;
    float4 kr[4];
    {
      const float* kp = kc + (size_t)min(jq, LMAX - 1) * 64 + qq * 16;
#pragma unroll
      for (int i = 0; i < 4; ++i) kr[i] = ldgf4(kp + 4 * i);
    }
    float vr[16];
#pragma unroll
    for (int i = 0; i < 16; ++i) vr[i] = ldg(vc + (size_t)min(wave + 16 * i, LMAX - 1) * 64 + lane);
#pragma unroll
    for (int i = 0; i < 4; ++i) pin(kr[i]);
#pragma unroll
    for (int i = 0; i < 16; ++i) pin(vr[i]);
    const uint32_t tg = c.tag(l, P_QKV);
    PD_MARK(l, 0);
    const bool ok = wait_tagged<1>(
        192, c, p.tq,
        [&](int i) { return i < 64 ? hq * 64 + i : i < 128 ? (NH + g) * 64 + (i - 64) : (NH + NKV + g) * 64 + (i - 128); },
        [=](int) { return tg; }, s.hin, s.flags);
    if (!ok) return false;
    PD_MARK(l, 1);
    if (tid < 64) {
      const int d = tid;
      qs[d] = rope1(s.hin, d, 32, cs, sn);
      kn[d] = rope1(s.hin + 64, d, 32, cs, sn);
      vn[d] = s.hin[128 + d];
      if (hq % rep == 0) {
        stg(kc + (size_t)pos * 64 + d, kn[d]);
        stg(vc + (size_t)pos * 64 + d, vn[d]);
      }
    }
    __syncthreads();
    PD_MARK(l, 3);
    // online softmax per wave: wave w takes positions cb + w + 16 i (i = lane / 4: four lanes
    // each for the scores) of every 256-position chunk, keeps its running maximum m, sum of
    // weights ws and weighted sum o (lane = dimension); the partials are combined once at the end.
    // The wave's positions below S are a prefix i < nw of its 16 (uniform).
    const float vnl = vn[lane];
    float m = -INFINITY, ws = 0.f, o = 0.f;
    for (int cb = 0; cb < S; cb += 256) {
      const int j = cb + jq, nw = min(16, max(0, (S - cb - wave + 15) / 16));
      if (nw == 0) break;  // uniform: no later chunk has positions of this wave either
      float a;
      if (cb == 0) {
        a = dot16(qs + qq * 16, kr);
      } else {
        float4 k4[4];
        const float* kp = kc + (size_t)min(j, LMAX - 1) * 64 + qq * 16;
#pragma unroll
        for (int i = 0; i < 4; ++i) k4[i] = ldgf4(kp + 4 * i);
        a = dot16(qs + qq * 16, k4);
      }
      if (j == pos) a = dot16(qs + qq * 16, reinterpret_cast<const float4*>(kn + qq * 16));  // one quad
      a = quad_sum(a);
      const float sc = j < S ? a * p.scale : -INFINITY;
      const float mn = fmaxf(m, wave_max(sc));  // finite: the wave has a position below S
      const float r = m == -INFINITY ? 0.f : expf(m - mn);
      const float pj = expf(sc - mn);
      ws = ws * r + wave_sum(qq == 0 ? pj : 0.f);
      o = o * r;
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        if (i < nw) {  // uniform
          const int jj = cb + wave + 16 * i;
          float v = cb == 0 ? vr[i] : ldg(vc + (size_t)jj * 64 + lane);
          if (jj == pos) v = vnl;  // uniform: the row is written this step
          o = fmaf(lane_at(pj, 4 * i), v, o);
        }
      }
      m = mn;
    }
    PD_MARK(l, 4);
    // the 16 waves' partials, combined in wave order: sum_w e_w o_w / sum_w e_w ws_w with
    // e_w = e^(m_w - M), lane w of wave 0 taking e_w (the next layer's reads of red and red16
    // follow its wait's barrier, which this wave joins only after the reads below)
    s.red[wave * 64 + lane] = o;
    if (lane == 0) {
      s.red16[wave] = m;
      s.red16[16 + wave] = ws;
    }
    __syncthreads();
    if (tid < 64) {
      const float mw = lane < kWaves ? s.red16[lane] : -INFINITY;
      const float mx = wave_max(mw);
      const float e = mw == -INFINITY ? 0.f : expf(mw - mx);
      const float den = wave_sum(lane < kWaves ? e * s.red16[16 + lane] : 0.f);
      float num = 0.f;
#pragma unroll
      for (int w = 0; w < kWaves; ++w) num = fmaf(lane_at(e, w), s.red[w * 64 + tid], num);
      tput(p.tatt + hq * 64 + tid, c.tag(l, P_ATT), num / den);
    }
    PD_MARK(l, 2);
  }
  return true;
}

// hmid(l) of columns [64 t, 64 t + 64): h(l) plus the o projection of all heads' outputs
// (K = NH * 64), a tile like the q|k|v one. h(l) of the chunk is waited for first (it is ready a
// whole head step earlier).
template <int SA, bool TR>
MIQ_PD_INLINE bool role_ored(const Params& p, const Ctx& c, const Lds& s, int t, int tok) {
  float zo = p.zoff;
  pin(zo);
  const int H = p.H, KO = p.NH * 64, c0 = t * kTile;
  for (int l = 0; l < p.L; ++l) {
    const uint64_t* lt = p.layers + (size_t)l * kSlots;
    Tile<__half, SA> w;
    tile_issue<__half, SA, true, true>(w, (const uint32_t*)lt[O_QW], (const uint32_t*)lt[O_QZ], (const __half*)lt[O_SC], H, c0, 0, KO / 32,
               p.lgs);
    float hres = 0.f;
    PD_MARK(l, 0);
    if (l == 0) {
      if (threadIdx.x < 64 && tok >= 0 && tok < p.V) hres = __half2float(p.embed[(size_t)tok * H + c0 + threadIdx.x]);
    } else {
      if (!wait_fixed<1>(kTile, c, fx_row(p, c.ep, l - 1, c0), p.ksd + 1, s.hin, s.flags)) return false;
      if (threadIdx.x < 64) hres = s.hin[threadIdx.x];
    }
    const uint32_t ta = c.tag(l, P_ATT);
    // (its own vote flags: the flags above may still be read by a slower wave)
    if (!wait_tagged<1>(
            KO, c, p.tatt, [](int i) { return i; }, [=](int) { return ta; }, s.xs, s.flags + kWaves))
      return false;
    PD_MARK(l, 1);
    const int ch = threadIdx.x;
    if (ch < KO / 8) {
      float v[8];
#pragma unroll
      for (int j = 0; j < 8; ++j) v[j] = s.xs[ch * 8 + j];
      stage_digits(ch, v, s.xa, s.cx);
    }
    __syncthreads();
    PD_MARK(l, 3);
    const float y = tile_sum(tile_mma_i8(w, s.xa, s.cx, 0, c0, p.lgs, zo), s.red);
    PD_MARK(l, 4);
    if (threadIdx.x < 64) tput(p.thmid + c0 + threadIdx.x, c.tag(l, P_HMID), hres + y);
    PD_MARK(l, 2);
    __syncthreads();
  }
  return true;
}

// gate|up projection, columns [64 t, 64 t + 64) of the interleaved 2I (gate 32 t .. + 31, up
// 32 t .. + 31): RMSNorm(hmid(l)) @ Wgu, published as silu(gate) * up. The tile also
// adds the residual hmid(l) of column chunks t, t + ngu, ... to h(l + 1) (term ksd).
template <int SA, bool TR>
MIQ_PD_INLINE bool role_gu(const Params& p, const Ctx& c, const Lds& s, int t) {
  float zo = p.zoff;
  pin(zo);
  const int H = p.H, N = 2 * p.I, c0 = t * kTile;
  for (int l = 0; l < p.L; ++l) {
    const uint64_t* lt = p.layers + (size_t)l * kSlots;
    Tile<__half, SA> w;
    tile_issue<__half, SA, true, true>(w, (const uint32_t*)lt[GU_QW], (const uint32_t*)lt[GU_QZ], (const __half*)lt[GU_SC], N, c0, 0, H / 32,
               p.lgs);
    float4 nw[2];
    norm_prefetch(nw, (const float*)lt[POST_LN], H);
    const uint32_t th = c.tag(l, P_HMID);
    PD_MARK(l, 0);
    if (!wait_tagged<1>(
            H, c, p.thmid, [&](int i) { return i; }, [=](int) { return th; }, s.xs, s.flags))
      return false;
    PD_MARK(l, 1);
    if (threadIdx.x < 64) {  // the residual hmid(l), term ksd of h(l + 1)
      const Fx hn = fx_row(p, c.ep, l);
      for (int k = t; k < H / kTile; k += p.ngu) fx_put(hn, k * kTile + threadIdx.x, s.xs[k * kTile + threadIdx.x], p.ksd);
    }
    const int ch = threadIdx.x;
    float v[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) v[j] = ch < H / 8 ? s.xs[ch * 8 + j] : 0.f;
    norm_stage(v, nw, s.red16);
    if (ch < H / 8) stage_digits(ch, v, s.xa, s.cx);
    __syncthreads();
    PD_MARK(l, 3);
    const float y = tile_sum(tile_mma_i8(w, s.xa, s.cx, 0, c0, p.lgs, zo), s.red);
    PD_MARK(l, 4);
    // the tile's columns are gate 32 t .. + 31 then up 32 t .. + 31 (the host interleaves the
    // weights' columns so): lane j < 32 of wave 0 pairs its gate with lane j + 32's up and
    // publishes silu(gate) * up, the down projection's input
    if (threadIdx.x < 64) {
      const float gu = y / norm_r(s.red16, H, p.eps);
      const float u = __shfl_down(gu, 32, 64);
      if (threadIdx.x < 32) tput(p.tgu + 32 * t + threadIdx.x, c.tag(l, P_GU), (gu * (1.f / (1.f + expf(-gu)))) * u);
    }
    PD_MARK(l, 2);
    __syncthreads();
  }
  return true;
}

// down projection, columns [64 t, 64 t + 64) of H over K-slice sl of I: the slice's share of
// silu(gate) * up @ Wd, term sl of h(l + 1).
template <int SD, bool TR>
MIQ_PD_INLINE bool role_down(const Params& p, const Ctx& c, const Lds& s, int t, int sl) {
  float zo = p.zoff;
  pin(zo);
  const int H = p.H, I = p.I, KS = I / p.ksd, rb = sl * (KS / 8), c0 = t * kTile;
  for (int l = 0; l < p.L; ++l) {
    const uint64_t* lt = p.layers + (size_t)l * kSlots;
    Tile<__half, SD> w;
    tile_issue<__half, SD, true, true>(w, (const uint32_t*)lt[D_QW], (const uint32_t*)lt[D_QZ], (const __half*)lt[D_SC], H, c0, rb, KS / 32,
               p.lgs);
    const uint32_t tg = c.tag(l, P_GU);
    PD_MARK(l, 0);
    if (!wait_tagged<2>(
            KS, c, p.tgu, [&](int i) { return sl * KS + i; }, [=](int) { return tg; }, s.hin, s.flags))
      return false;
    PD_MARK(l, 1);
    const int ch = threadIdx.x;
    if (ch < KS / 8) {
      float v[8];
#pragma unroll
      for (int j = 0; j < 8; ++j) v[j] = s.hin[ch * 8 + j];
      stage_digits(ch, v, s.xa, s.cx);
    }
    __syncthreads();
    PD_MARK(l, 3);
    const float y = tile_sum(tile_mma_i8(w, s.xa, s.cx, rb, c0, p.lgs, zo), s.red);
    PD_MARK(l, 4);
    if (threadIdx.x < 64 && c0 + (int)threadIdx.x < H) fx_put(fx_row(p, c.ep, l), c0 + threadIdx.x, y, sl);
    PD_MARK(l, 2);
    __syncthreads();
  }
  return true;
}

// Tied head over 64-column tiles b, b + G, ... (the next tile's loads issued before the current
// one is computed) with a running arg-max, published as tagged (value, index) words.
template <int SA, bool TR>
MIQ_PD_INLINE bool role_head(const Params& p, const Ctx& c, const Lds& s, int tok) {
  const int H = p.H, V = p.V, G = gridDim.x, b = blockIdx.x;
  const int ntile = (V + kTile - 1) / kTile;
  float zo = p.head_zoff;
  pin(zo);
  // three tiles in flight: b and b + G are loaded before the wait for h; then each step issues
  // the tile two steps ahead (not pinned: the step's barrier keeps the loads where they are
  // issued, and a pin would wait for them a step early)
  Tile<float, SA> t0, t1, t2;
  if (b < ntile) tile_issue<float, SA, true, true>(t0, p.head_qw, p.head_qz, p.head_sc, V, b * kTile, 0, H / 32, p.lgs);
  if (b + G < ntile) tile_issue<float, SA, true, true>(t1, p.head_qw, p.head_qz, p.head_sc, V, (b + G) * kTile, 0, H / 32, p.lgs);
  float4 nw[2];
  norm_prefetch(nw, p.final_norm, H);
  PD_MARK(p.L, 0);
  float v[8];
  if (!gather_h(p, c, s, p.L, tok, s.hin, v)) return false;
  PD_MARK(p.L, 1);
  const int ch = threadIdx.x;
  norm_stage(v, nw, s.red16);
  if (ch < H / 8) stage_digits(ch, v, s.xa, s.cx);
  __syncthreads();
  const float rn = norm_r(s.red16, H, p.eps);
  float bv = -INFINITY;
  int bi = 0x7fffffff;
  auto step = [&](Tile<float, SA>& cur, Tile<float, SA>& ahead, int t)
                  __attribute__((always_inline)) {
    if (t >= ntile) return;  // uniform
    if (t + 2 * G < ntile)
      tile_issue<float, SA, false, true>(ahead, p.head_qw, p.head_qz, p.head_sc, V, (t + 2 * G) * kTile, 0, H / 32, p.lgs);
    const int n = t * kTile + (int)threadIdx.x;
    const float y = tile_sum(tile_mma_i8(cur, s.xa, s.cx, 0, t * kTile, p.lgs, zo), s.red) / rn;
    if (threadIdx.x < 64 && n < V) {
      p.logits[n] = y;
      if (better(y, n, bv, bi) || (bv != bv && y == y)) { bv = y; bi = n; }
    }
    __syncthreads();
  };
  for (int t = b; t < ntile; t += 3 * G) {
    step(t0, t2, t);
    step(t1, t0, t + G);
    step(t2, t1, t + 2 * G);
  }
  if (threadIdx.x < 64) {
    wave_argmax(bv, bi);
    if (threadIdx.x == 0) {
      tput(p.tamax + b, c.tag(p.L, P_AMAX), bv);
      tput(p.tamax + G + b, c.tag(p.L, P_AMAX), __int_as_float(bi));
    }
  }
  PD_MARK(p.L, 2);
  return true;
}

// Workgroup 0: combine the G arg-max partials, emit the token and advance the decode state.
MIQ_PD_INLINE bool finish_token(const Params& p, const Ctx& c, const Lds& s, int pos) {
  const int G = gridDim.x;
  const uint32_t tg = c.tag(p.L, P_AMAX);
  if (!wait_tagged<1>(
          2 * G, c, p.tamax, [&](int i) { return i; }, [=](int) { return tg; }, s.hin, s.flags))
    return false;
  if (threadIdx.x < 64) {
    float fv = -INFINITY;
    int fi = 0x7fffffff;
    for (int gi = threadIdx.x; gi < G; gi += 64) {
      const float v = s.hin[gi];
      const int i = __float_as_int(s.hin[G + gi]);
      if (better(v, i, fv, fi) || (fv != fv && v == v)) { fv = v; fi = i; }
    }
    wave_argmax(fv, fi);
    if (threadIdx.x == 0) {
      if (fi >= p.V) fi = 0;  // all logits NaN
      p.ids[0] = fi;
      const int step = p.state[1];
      if (step < p.hist_len) p.history[step] = fi;
      p.state[1] = step + 1;
      p.state[3] = fi;
      p.state[0] = pos + 1;
      p.ctl[0] = c.ep;
    }
  }
  return true;
}

template <int SA, int SD, bool TR>
__global__ __launch_bounds__(kThreads) void decode_persistent_kernel(Params p) {
  extern __shared__ __align__(16) float lds[];
  Lds s;
  s.hin = lds;
  s.xs = s.hin + p.lds_a;
  s.xa = reinterpret_cast<unsigned char*>(s.xs + p.lds_x);
  s.cx = reinterpret_cast<float2*>(s.xa + (size_t)(p.lds_x / 32) * kStep8Bytes);
  s.red = reinterpret_cast<float*>(s.cx + p.lds_x / 32);
  s.red16 = s.red + kKParts * 64;
  s.qkv = s.red16 + 32;
  s.flags = reinterpret_cast<int*>(s.qkv + kQkvFloats);
  Ctx c;
  c.deadline = wall_clock64() + p.spin_limit;
  PD_MARK(p.L + 1, 0);
  c.ep = p.ctl[0] + 1u;
  c.L = p.L;
  const int pos = p.state[0];
  const int tok = p.ids[0];
  if (pos < 0 || pos >= p.LMAX) {  // uniform over the grid: every workgroup leaves at once
    if (blockIdx.x == 0 && threadIdx.x == 0) atomicOr(p.ctl + 1, 2u);
    return;
  }
  // After a timed-out step the exchange words and fixed-point banks are dirty (its epoch is
  // reused), so every later step leaves at entry without touching the decode state until the
  // workspace is reset; the host then finishes the sequence with the launch sequence. One
  // thread reads the bit and the workgroup follows it, so its waves cannot split on it.
  if (threadIdx.x == 0) s.flags[0] = (int)__hip_atomic_load(p.ctl + 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  __syncthreads();
  const bool failed_before = s.flags[0] & 1;
  __syncthreads();
  if (failed_before) return;
  {  // the next token's bank back to zero (this token's was zeroed by the previous step)
    unsigned long long* z = p.fx + ((c.ep + 1u) & 1u) * p.bank_words;
    for (size_t i = (size_t)blockIdx.x * kThreads + threadIdx.x; i < p.bank_words; i += (size_t)gridDim.x * kThreads)
      __hip_atomic_store(z + i, 0ull, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
  int r = blockIdx.x;
  bool ok = true;
  if (r < p.nq) {
    ok = role_qkv<SA, TR>(p, c, s, r, tok);
  } else if ((r -= p.nq) < p.na) {
    ok = role_attn<TR>(p, c, s, r, pos);
  } else if ((r -= p.na) < p.no) {
    ok = role_ored<SA, TR>(p, c, s, r, tok);
  } else if ((r -= p.no) < p.ngu) {
    ok = role_gu<SA, TR>(p, c, s, r);
  } else if ((r -= p.ngu) < p.nd) {
    ok = role_down<SD, TR>(p, c, s, r % p.no, r / p.no);
  }
  ok = ok && role_head<SA, TR>(p, c, s, tok);
  if (ok && blockIdx.x == 0) ok = finish_token(p, c, s, pos);
  if (!ok && threadIdx.x == 0) atomicOr(p.ctl + 1, 1u);
  PD_MARK(p.L + 1, 1);
}

// Role counts, K-slices of the down projection and LDS regions for a model shape.
struct Plan {
  int G, nq, na, no, ngu, ksd, nd, lds_a, lds_x, spa, spd;
  size_t lds_bytes, ws_bytes, bank_words;
  size_t off_tq, off_tatt, off_thmid, off_tgu, off_tamax, off_fx, off_side;
};

static int plan(int L, int H, int NH, int NKV, int HD, int I, int V, int LMAX, int gs, int bits, Plan* pl) {
  MIQ_REQUIRE(L > 0 && H > 0 && NH > 0 && NKV > 0 && NH % NKV == 0 && I > 0 && V > 0 && LMAX > 0 && gs > 0,
              MIQ_ERR_INVALID, "decode_persistent: L=%d H=%d NH=%d NKV=%d I=%d V=%d LMAX=%d gs=%d", L, H, NH, NKV, I, V,
              LMAX, gs);
  MIQ_REQUIRE(bits == 4 && HD == 64, MIQ_ERR_UNSUPPORTED, "decode_persistent: needs int4 and head dim 64 (bits=%d HD=%d)",
              bits, HD);
  const int NQ = (NH + 2 * NKV) * HD, NHD = NH * HD;
  MIQ_REQUIRE(H % kTile == 0 && NQ % kTile == 0 && (2 * I) % kTile == 0 && gs >= 64 && (gs & (gs - 1)) == 0 &&
                  V % 8 == 0,
              MIQ_ERR_UNSUPPORTED,
              "decode_persistent: H, q|k|v width and 2I must be multiples of 64, gs a power of two >= 64, V of 8");
  MIQ_REQUIRE(H % gs == 0 && NHD % gs == 0 && I % gs == 0, MIQ_ERR_UNSUPPORTED,
              "decode_persistent: H, NH*HD and I must be multiples of the group size %d", gs);
  // K in 64-value steps (the int8 digit tile), at most kMaxSPQ / 2 per k-part of a tile
  auto rows_ok = [&](int K) { return K % 64 == 0 && K <= 32 * kKParts * kMaxSPQ; };
  MIQ_REQUIRE(rows_ok(H) && H <= kThreads && LMAX <= 8192 && NHD <= kThreads &&
                  NHD % 64 == 0 && (NHD / 64 + kKParts - 1) / kKParts <= (H / 64 + kKParts - 1) / kKParts,
              MIQ_ERR_UNSUPPORTED, "decode_persistent: H=%d / NH=%d / LMAX=%d out of range", H, NH, LMAX);
  int cus = 0, dev = 0;
  if (hipGetDevice(&dev) != hipSuccess ||
      hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus <= 0)
    return fail(MIQ_ERR_HIP, "decode_persistent: cannot query the CU count");
  Plan q{};
  q.G = cus;
  q.nq = NQ / kTile;
  q.na = NH;
  q.no = H / kTile;
  q.ngu = 2 * I / kTile;
  q.ksd = 0;
  for (int k = 8; k >= 1; k >>= 1) {
    if (I % (64 * k) || !rows_ok(I / k) || 2 * (I / k) > 4 * kThreads) continue;
    if (q.nq + q.na + q.no + q.ngu + q.no * k > q.G) continue;
    q.ksd = k;
    break;
  }
  MIQ_REQUIRE(q.ksd > 0 && 2 * q.G <= kThreads && NH * kTile <= 2 * kThreads, MIQ_ERR_UNSUPPORTED,
              "decode_persistent: the roles of this shape do not fit %d workgroups", q.G);
  q.nd = q.no * q.ksd;
  const int KS = I / q.ksd;
  q.spa = 2 * ((H / 64 + kKParts - 1) / kKParts);  // 32-k halves per k-part (64-k steps dealt whole)
  q.spd = 2 * ((KS / 64 + kKParts - 1) / kKParts);
  // hin: exchange words of every role (the heads' q|k|v words: 192), the arg-max partials (2G)
  q.lds_a = std::max(std::max(std::max(H, 2 * KS), (NH + 1) * kTile), std::max(192, 2 * q.G));
  q.lds_a = (q.lds_a + 3) & ~3;
  q.lds_x = (std::max(std::max(H, KS), NHD) + 63) & ~63;  // even step count: red 16-byte aligned
  q.lds_bytes = (size_t)(q.lds_a + q.lds_x) * 4 + (size_t)(q.lds_x / 32) * kStep8Bytes +
                (size_t)(2 * (q.lds_x / 32) + kKParts * 64 + 32 + kQkvFloats + 2 * kWaves) * 4;
  int lds_max = 0;
  if (hipDeviceGetAttribute(&lds_max, hipDeviceAttributeMaxSharedMemoryPerBlock, dev) != hipSuccess || lds_max <= 0)
    return fail(MIQ_ERR_HIP, "decode_persistent: cannot query the LDS limit");
  MIQ_REQUIRE(q.lds_bytes <= (size_t)lds_max, MIQ_ERR_UNSUPPORTED,
              "decode_persistent: %zu bytes of LDS for this shape exceed the device's %d", q.lds_bytes, lds_max);
  size_t off = 256;  // control words
  auto take = [&](size_t bytes) {
    const size_t o = off;
    off += (bytes + 255) & ~(size_t)255;
    return o;
  };
  q.off_tq = take((size_t)NQ * 8);
  q.off_tatt = take((size_t)NH * 64 * 8);
  q.off_thmid = take((size_t)H * 8);
  q.off_tgu = take((size_t)I * 8);
  q.off_tamax = take(2 * (size_t)q.G * 8);
  const size_t n = (size_t)L * H;  // h(l + 1) words of every layer
  q.bank_words = ((n * 12 + 255) & ~(size_t)255) / 8;
  q.off_fx = take(2 * q.bank_words * 8);
  q.off_side = take((size_t)(q.ksd + 1) * n * 4);
  q.ws_bytes = off;
  *pl = q;
  return MIQ_OK;
}

}  // namespace pd
}  // namespace miq

using namespace miq;

extern "C" int miq_decode_persistent_plan(int L, int H, int NH, int NKV, int HD, int I, int V, int LMAX, int gs,
                                          int bits, int* grid, size_t* ws_bytes) {
  pd::Plan pl;
  const int rc = pd::plan(L, H, NH, NKV, HD, I, V, LMAX, gs, bits, &pl);
  if (rc != MIQ_OK) return rc;
  if (grid) *grid = pl.G;
  if (ws_bytes) *ws_bytes = pl.ws_bytes;
  return MIQ_OK;
}

static int decode_persistent(const uint64_t* layer_table, const void* embed, const int32_t* head_qweight,
                             const int32_t* head_qzeros, const float* head_scales, const float* final_norm,
                             const float* cos_tab, const float* sin_tab, int32_t* ids, int32_t* history, int hist_len,
                             int32_t* state, float* logits, void* ws, size_t ws_bytes, int L, int H, int NH, int NKV,
                             int HD, int I, int V, int LMAX, int gs, int bits, float eps, float zoff, float head_zoff,
                             void* stream, uint64_t* trace) {
  pd::Plan pl;
  const int rc = pd::plan(L, H, NH, NKV, HD, I, V, LMAX, gs, bits, &pl);
  if (rc != MIQ_OK) return rc;
  MIQ_REQUIRE(layer_table && embed && head_qweight && head_qzeros && head_scales && final_norm && cos_tab && sin_tab &&
                  ids && state && logits && ws && (history || hist_len == 0) && hist_len >= 0,
              MIQ_ERR_INVALID, "decode_persistent: null pointer");
  MIQ_REQUIRE(ws_bytes >= pl.ws_bytes, MIQ_ERR_INVALID, "decode_persistent: workspace %zu bytes, need %zu", ws_bytes,
              pl.ws_bytes);
  MIQ_REQUIRE(aligned(ws, 256) && aligned(layer_table, 8), MIQ_ERR_ALIGN,
              "decode_persistent: workspace must be 256-byte aligned");
  int dev = 0, per_cu = 0, khz = 0;
  // 32-k steps per k-part (wave) of the K = H projections and of a down K-slice, rounded up to the
  // instantiated register capacities
  void (*kfn)(pd::Params) = nullptr;
  // (H <= 1024 keeps spa <= 2)
  if (pl.spd <= 4) kfn = trace ? pd::decode_persistent_kernel<2, 4, true> : pd::decode_persistent_kernel<2, 4, false>;
  else kfn = trace ? pd::decode_persistent_kernel<2, 8, true> : pd::decode_persistent_kernel<2, 8, false>;
  auto kern = reinterpret_cast<const void*>(kfn);
  if (hipGetDevice(&dev) != hipSuccess ||
      hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, kern, pd::kThreads, pl.lds_bytes) != hipSuccess)
    return fail(MIQ_ERR_HIP, "decode_persistent: occupancy query failed");
  MIQ_REQUIRE(per_cu >= 1, MIQ_ERR_UNSUPPORTED, "decode_persistent: a workgroup does not fit a CU");
  if (hipDeviceGetAttribute(&khz, hipDeviceAttributeWallClockRate, dev) != hipSuccess || khz <= 0) khz = 100000;
  pd::Params p{};
  unsigned char* w = static_cast<unsigned char*>(ws);
  p.layers = layer_table;
  p.embed = static_cast<const __half*>(embed);
  p.head_qw = reinterpret_cast<const uint32_t*>(head_qweight);
  p.head_qz = reinterpret_cast<const uint32_t*>(head_qzeros);
  p.head_sc = head_scales;
  p.final_norm = final_norm;
  p.cos_t = cos_tab;
  p.sin_t = sin_tab;
  p.ids = ids;
  p.history = history;
  p.state = state;
  p.logits = logits;
  p.ctl = reinterpret_cast<uint32_t*>(w);
  p.tq = reinterpret_cast<uint64_t*>(w + pl.off_tq);
  p.tatt = reinterpret_cast<uint64_t*>(w + pl.off_tatt);
  p.thmid = reinterpret_cast<uint64_t*>(w + pl.off_thmid);
  p.tgu = reinterpret_cast<uint64_t*>(w + pl.off_tgu);
  p.tamax = reinterpret_cast<uint64_t*>(w + pl.off_tamax);
  p.fx = reinterpret_cast<unsigned long long*>(w + pl.off_fx);
  p.fside = reinterpret_cast<float*>(w + pl.off_side);
  p.bank_words = pl.bank_words;
  p.L = L;
  p.H = H;
  p.NH = NH;
  p.NKV = NKV;
  p.I = I;
  p.V = V;
  p.LMAX = LMAX;
  p.gs = gs;
  p.lgs = 0;
  while ((1 << p.lgs) < gs) ++p.lgs;
  p.hist_len = hist_len;
  p.ksd = pl.ksd;
  p.nq = pl.nq;
  p.na = pl.na;
  p.no = pl.no;
  p.ngu = pl.ngu;
  p.nd = pl.nd;
  p.lds_a = pl.lds_a;
  p.lds_x = pl.lds_x;
  p.eps = eps;
  p.scale = 1.0f / sqrtf((float)HD);
  p.zoff = zoff;
  p.head_zoff = head_zoff;
  p.trace = reinterpret_cast<unsigned long long*>(trace);
  p.spin_limit = (long long)khz * 100;  // 100 ms
  if (const char* e = getenv("MIQ_PD_SPIN_TICKS")) {  // a shorter bound, for tests of the error path
    const long long t = atoll(e);
    if (t > 0 && t < p.spin_limit) p.spin_limit = t;
  }
  hipLaunchKernelGGL(kfn, dim3(pl.G), dim3(pd::kThreads), pl.lds_bytes,
                     static_cast<hipStream_t>(stream), p);
  return check_launch("decode_persistent");
}

extern "C" int miq_decode_persistent(const uint64_t* layer_table, const void* embed, const int32_t* head_qweight,
                                     const int32_t* head_qzeros, const float* head_scales, const float* final_norm,
                                     const float* cos_tab, const float* sin_tab, int32_t* ids, int32_t* history,
                                     int hist_len, int32_t* state, float* logits, void* ws, size_t ws_bytes, int L,
                                     int H, int NH, int NKV, int HD, int I, int V, int LMAX, int gs, int bits, float eps,
                                     float zoff, float head_zoff, void* stream) {
  return decode_persistent(layer_table, embed, head_qweight, head_qzeros, head_scales, final_norm, cos_tab, sin_tab, ids,
                           history, hist_len, state, logits, ws, ws_bytes, L, H, NH, NKV, HD, I, V, LMAX, gs, bits, eps,
                           zoff, head_zoff, stream, nullptr);
}

extern "C" int miq_decode_persistent_trace(const uint64_t* layer_table, const void* embed, const int32_t* head_qweight,
                                           const int32_t* head_qzeros, const float* head_scales,
                                           const float* final_norm, const float* cos_tab, const float* sin_tab,
                                           int32_t* ids, int32_t* history, int hist_len, int32_t* state, float* logits,
                                           void* ws, size_t ws_bytes, int L, int H, int NH, int NKV, int HD, int I, int V,
                                           int LMAX, int gs, int bits, float eps, float zoff, float head_zoff,
                                           uint64_t* trace, size_t trace_words, void* stream) {
  int grid = 0;
  const int rc = miq_decode_persistent_plan(L, H, NH, NKV, HD, I, V, LMAX, gs, bits, &grid, nullptr);
  if (rc != MIQ_OK) return rc;
  MIQ_REQUIRE(trace && aligned(trace, 8), MIQ_ERR_INVALID, "decode_persistent_trace: null or unaligned trace buffer");
  MIQ_REQUIRE(trace_words >= (size_t)grid * (L + 2) * 8, MIQ_ERR_INVALID,
              "decode_persistent_trace: trace holds %zu words, need %zu", trace_words, (size_t)grid * (L + 2) * 8);
  return decode_persistent(layer_table, embed, head_qweight, head_qzeros, head_scales, final_norm, cos_tab, sin_tab, ids,
                           history, hist_len, state, logits, ws, ws_bytes, L, H, NH, NKV, HD, I, V, LMAX, gs, bits, eps,
                           zoff, head_zoff, stream, trace);
}
