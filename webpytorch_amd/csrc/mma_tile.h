// Exact int4 GPTQ tiles on the gfx950 matrix cores for one row of fp32 activations, shared by
// the persistent decode step and the one-row GEMV.
#pragma once
#include "miq_common.h"

namespace miq {
namespace mt {

// The thread index as a value the compiler cannot see through: index math derived from it is
// recomputed where it is used (a few instructions per layer) instead of being hoisted out of
// the layer loop and held in registers for the whole token.
__device__ __forceinline__ int opaque_tid() {
  int v = threadIdx.x;
  asm volatile("" : "+v"(v));
  return v;
}

// ---- 64-column int4 tiles on the matrix cores ---------------------------------------------
// A tile of 64 columns is computed by the 16 waves of a workgroup, each taking all 64 columns
// and one k-part (a sixteenth) of the steps: lane l loads 16 bytes of packed row (l >> 4) of
// each 32-k step -- columns 4 (l & 15) .. + 3 -- and feeds MFMA t the word of column
// 4 (l & 15) + t, which holds exactly its B fragment (column l & 15 of MFMA t, the 8 codes of
// packed row l >> 4). The four MFMAs of a step share the A fragment, so the per-step work (A
// read, sums, addresses) is paid once per four MFMAs. The products themselves run on the int8
// matrix cores (tile_mma_i8 below).

// Raw scale bits of 4 adjacent columns (fp16: 8 bytes, fp32: 16 bytes), converted when used.
template <typename ST> struct Scales4;
template <> struct Scales4<__half> {
  using T = uint2;
  static __device__ __forceinline__ T load(const __half* p) { return ldg2(p); }
  static __device__ __forceinline__ float get(const T& v, int t) {
    const uint32_t w = t < 2 ? v.x : v.y;
    return __half2float(__ushort_as_half((unsigned short)((t & 1) ? w >> 16 : w & 0xFFFFu)));
  }
};
template <> struct Scales4<float> {
  using T = uint4;
  static __device__ __forceinline__ T load(const float* p) { return ldg4(p); }
  static __device__ __forceinline__ float get(const T& v, int t) {
    return __uint_as_float(t == 0 ? v.x : t == 1 ? v.y : t == 2 ? v.z : v.w);
  }
};

constexpr int kKParts = 16;  // k-parts of a tile: the waves of a 1024-thread workgroup

template <typename ST, int SPQ>
struct Tile {
  uint4 w[SPQ];                    // codes of 4 adjacent columns, one packed row per step
  uint32_t z[SPQ];                 // zero-point word of those columns' group
  typename Scales4<ST>::T s[SPQ];  // raw scale bits of the 4 columns
  int st0, ns;                     // first step and step count of this wave
};

// Holds loaded values in registers from here on. Without it the compiler sinks loads issued
// ahead of a wait down to their first use after the wait, which puts a memory round trip back
// on the critical path; the empty asm makes the values used (so loaded) at this point.
__device__ __forceinline__ void pin(float& v) { asm volatile("" : "+v"(v)); }
__device__ __forceinline__ void pin(uint32_t& v) { asm volatile("" : "+v"(v)); }
__device__ __forceinline__ void pin(float4& v) { asm volatile("" : "+v"(v.x), "+v"(v.y), "+v"(v.z), "+v"(v.w)); }
__device__ __forceinline__ void pin(uint4& v) { asm volatile("" : "+v"(v.x), "+v"(v.y), "+v"(v.z), "+v"(v.w)); }
__device__ __forceinline__ void pin(uint2& v) { asm volatile("" : "+v"(v.x), "+v"(v.y)); }
template <typename ST, int SPQ>
__device__ __forceinline__ void pin(Tile<ST, SPQ>& t) {
#pragma unroll
  for (int i = 0; i < SPQ; ++i) {
    pin(t.w[i]);
    pin(t.z[i]);
    pin(t.s[i]);
  }
}

// Issues this wave's loads for the tile of columns [c0, c0 + 64) (clamped to N - 4; N a
// multiple of 4) over the nsteps 32-k steps starting at packed row rb (absolute, for the group
// index; groups are 2^lgs values, 2^(lgs - 3) packed rows). nsteps <= kKParts * SPQ.
// PAIRS: steps are dealt to waves two at a time (the 64-k steps of the int8 digit tile; nsteps
// even).
template <typename ST, int SPQ, bool PIN = true, bool PAIRS = false>
__device__ __forceinline__ void tile_issue(Tile<ST, SPQ>& t, const uint32_t* qw, const uint32_t* qz, const ST* sc,
                                           int N, int c0, int rb, int nsteps, int lgs) {
  const int tid = opaque_tid();
  const int wave = uniform(tid >> 6), lane = tid & 63;
  // contiguous step ranges, the first nsteps % kKParts waves one step longer: wave w runs on
  // SIMD w % 4, so every SIMD gets the same step count to within one
  const int units = PAIRS ? nsteps >> 1 : nsteps, per = PAIRS ? 2 : 1;
  const int base = units / kKParts, extra = units % kKParts;
  t.st0 = per * (wave * base + min(wave, extra));
  t.ns = per * (base + (wave < extra ? 1 : 0));
  const int c = min(c0 + 4 * (lane & 15), N - 4);
  const int r0 = rb + 4 * t.st0, gsh = lgs - 3;
  const uint32_t* wp = qw + (uint32_t)((r0 + (lane >> 4)) * N + c);
  if (t.ns > 0) {
    // unguarded loads (steps past the wave's last repeat it) issue back to back
#pragma unroll
    for (int i = 0; i < SPQ; ++i) {
      const int ii = min(i, t.ns - 1);
      const int g = (r0 + 4 * ii) >> gsh;
      t.w[i] = ldg4(wp + (uint32_t)(4 * ii * N));
      t.s[i] = Scales4<ST>::load(sc + (uint32_t)(g * N + c));
      t.z[i] = ldg(qz + (uint32_t)(g * (N >> 3) + (c >> 3)));
    }
    if (PIN) pin(t);
  }
}

// Sums the kKParts k-parts of each column in wave order; valid in threads 0..63 (column
// c0 + thread). red holds kKParts x 64 floats, 16-byte aligned.
__device__ __forceinline__ float tile_sum(float4 acc, float* red) {
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  if (lane < 16) *reinterpret_cast<float4*>(red + wave * 64 + 4 * lane) = acc;
  __syncthreads();
  float y = 0.f;
  if (threadIdx.x < 64) {
#pragma unroll
    for (int q = 0; q < kKParts; ++q) y += red[q * 64 + threadIdx.x];
  }
  return y;
}

// ---- 64-column int4 tile on the int8 matrix cores ----------------------------------------
// v_mfma_i32_16x16x64_i8 (64 k per instruction, of which rows 0-3 are used) with 2 VALU per
// packed word for the B operand. (An earlier form split fp32 x exactly into three bf16 terms for
// v_mfma_f32_16x16x32_bf16: twice the matrix-core instructions per k and 7 VALU per packed word
// to build bf16 codes; the decode token went 387 -> 359 us with this one.) Each 64-k step of x
// is held in fixed point at the step's own
// scale: with 2^e > max |x| over the step, X = rint(x 2^(30 - e)) (|X| <= 2^30; the rounding
// error is at most 2^-31 of the step's largest value), split into four signed 8-bit digits,
// X = d0 + 2^8 d1 + 2^16 d2 + 2^24 d3 (|d3| <= 64), which are rows 0-3 of A. B holds the codes as
// int8 (0..15). Row t of D is then the exact integer sum_k d_t c_k, and a step's products are
// 2^(e - 30) (D0 + 2^8 D1 + 2^16 D2 + 2^24 D3), formed in fp32 from two exact int32 halves.
// Zero points use the step's fp32 sum of x. A step holding NaN or an
// infinity stores a NaN scale, so its outputs are NaN.
//
// A 64-k step of A is 4 lane groups x 4 digit rows x 16 bytes (272 with padding). Lane l (row
// l % 16, group g = l / 16) reads bytes 16 g .. + 15 of its row, matching its B bytes: the low
// nibbles of packed row g of the step's first 32-k half (codes 0, 2, 4, 6 of the row), its high
// nibbles (1, 3, 5, 7), then the same two of packed row g of the second half. Staging thread ch
// (chunk u = ch % 8 of step ch / 8) writes its 8 values in that order to group u % 4, bytes
// 8 (u / 4) .. + 7.
constexpr int kStep8Bytes = 272;
typedef int i32x4 __attribute__((ext_vector_type(4)));

// Rows of a 4 x 4 byte matrix given as columns: a, b, c, d each hold one value's four digits
// (byte t = digit t); r[t] gets digit t of a, b, c, d in bytes 0-3.
__device__ __forceinline__ void transpose4(uint32_t a, uint32_t b, uint32_t c, uint32_t d, uint32_t* r) {
  const uint32_t t0 = __builtin_amdgcn_perm(b, a, 0x05010400u), t1 = __builtin_amdgcn_perm(b, a, 0x07030602u);
  const uint32_t t2 = __builtin_amdgcn_perm(d, c, 0x05010400u), t3 = __builtin_amdgcn_perm(d, c, 0x07030602u);
  r[0] = __builtin_amdgcn_perm(t2, t0, 0x05040100u);
  r[1] = __builtin_amdgcn_perm(t2, t0, 0x07060302u);
  r[2] = __builtin_amdgcn_perm(t3, t1, 0x05040100u);
  r[3] = __builtin_amdgcn_perm(t3, t1, 0x07060302u);
}

// Stages chunk ch of K / 8 (8 values) of the digit tile's A operand; the eight chunks of a step
// (consecutive threads, all present since K % 64 == 0) combine their maxima and sums, and the
// first writes cx[step] = (2^(e - 30) or NaN, sum of the step's x). The largest |x| is taken on
// the bit patterns (ordered like the magnitudes; NaN and infinities above every finite value).
// The signed digits of X (each in [-128, 127], the top one within +-64) are the bytes of
// (X + 0x80808080) ^ 0x80808080: adding 128 to every digit makes them the unsigned bytes of
// X + 0x80808080, which stays within 32 bits.
__device__ __forceinline__ void stage_digits(int ch, const float* v, unsigned char* xa, float2* cx) {
  uint32_t mb = 0u;
#pragma unroll
  for (int j = 0; j < 8; ++j) mb = max(mb, __float_as_uint(v[j]) & 0x7FFFFFFFu);
  mb = max(mb, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)mb, 0xB1, 0xF, 0xF, false));
  mb = max(mb, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)mb, 0x4E, 0xF, 0xF, false));
  mb = max(mb, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)mb, 0x141, 0xF, 0xF, false));  // the step's 8 lanes
  const bool ok = mb < 0x7F800000u;
  int e = 0;
  if (ok && mb) (void)frexpf(__uint_as_float(mb), &e);  // max |x| < 2^e
  uint32_t w[8];
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    const int X = ok ? (int)rintf(ldexpf(v[j], 30 - e)) : 0;
    w[j] = ((uint32_t)X + 0x80808080u) ^ 0x80808080u;
  }
  uint32_t ev[4], od[4];
  transpose4(w[0], w[2], w[4], w[6], ev);
  transpose4(w[1], w[3], w[5], w[7], od);
  const int u = ch & 7;
  unsigned char* dst = xa + (ch >> 3) * kStep8Bytes + (u & 3) * 64 + (u >> 2) * 8;
#pragma unroll
  for (int r = 0; r < 4; ++r) *reinterpret_cast<uint2*>(dst + 16 * r) = make_uint2(ev[r], od[r]);
  float sm = ((v[0] + v[1]) + (v[2] + v[3])) + ((v[4] + v[5]) + (v[6] + v[7]));
  sm += dpp_move<0xB1>(sm);
  sm += dpp_move<0x4E>(sm);
  sm += dpp_move<0x141>(sm);
  if (u == 0) cx[ch >> 3] = make_float2(ok ? ldexpf(1.f, e - 30) : __builtin_nanf(""), sm);
}

// This wave's share of sum_k x_k W[k][c] for its 4 columns (lanes 0..15: columns c0 + 4 lane + t)
// from the digit-staged A. The tile's steps are 32-k halves dealt in pairs (tile_issue PAIRS);
// each pair is one 64-k step. Quantization groups are at least 64 values.
template <typename ST, int SPQ>
__device__ __forceinline__ float4 tile_mma_i8(const Tile<ST, SPQ>& t, const unsigned char* xa, const float2* cx,
                                              int rb, int c0, int lgs, float zoff) {
  float acc[4] = {0.f, 0.f, 0.f, 0.f};
  if (t.ns == 0) return make_float4(0.f, 0.f, 0.f, 0.f);  // wave-uniform
  const int tid = opaque_tid();
  const int lane = tid & 63;
  const int sh = ((c0 + 4 * (lane & 15)) & 7) * 4;
  const bool arow = (lane & 15) < 4;  // only D rows 0-3 are read
  const int s0 = t.st0 >> 1, n8 = t.ns >> 1;
  const unsigned char* ap = xa + s0 * kStep8Bytes + (lane >> 4) * 64 + (lane & 15) * 16;
  uint32_t mk = 0x0F0F0F0Fu;
  asm volatile("" : "+v"(mk));
  const int r0 = rb + 4 * t.st0, gsh = lgs - 3;
  float pg[4] = {0.f, 0.f, 0.f, 0.f};  // the current group's products
  float xs = 0.f;
#pragma unroll
  for (int i = 0; i < SPQ / 2; ++i) {
    if (i < n8) {
      i32x4 a = {0, 0, 0, 0};
      if (arow) a = *reinterpret_cast<const i32x4*>(ap + i * kStep8Bytes);
      const float2 xc = cx[s0 + i];
      const uint4 wa = t.w[2 * i], wb = t.w[2 * i + 1];
      const uint32_t qa[4] = {wa.x, wa.y, wa.z, wa.w}, qb[4] = {wb.x, wb.y, wb.z, wb.w};
      i32x4 dq[4];
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const i32x4 b = {(int)(qa[q] & mk), (int)((qa[q] >> 4) & mk), (int)(qb[q] & mk), (int)((qb[q] >> 4) & mk)};
        dq[q] = __builtin_amdgcn_mfma_i32_16x16x64_i8(a, b, (i32x4){0, 0, 0, 0}, 0, 0, 0);
      }
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int lo = dq[q][0] + (dq[q][1] << 8), hi = dq[q][2] + (dq[q][3] << 8);
        pg[q] = fmaf(fmaf((float)hi, 65536.f, (float)lo), xc.x, pg[q]);
      }
      xs += xc.y;
      const int r = r0 + 8 * i;
      if (i + 1 == n8 || ((r + 8) >> gsh) != (r >> gsh)) {  // last step of this group
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const float zc = (float)((t.z[2 * i] >> (sh + 4 * q)) & 15u) + zoff;
          acc[q] = fmaf(Scales4<ST>::get(t.s[2 * i], q), pg[q] - zc * xs, acc[q]);
          pg[q] = 0.f;
        }
        xs = 0.f;
      }
    }
  }
  return make_float4(acc[0], acc[1], acc[2], acc[3]);
}

// ---- deterministic split-K sums in fixed point ------------------------------------------
// The K-slices of one output meet in a zeroed 64-bit word: each adds its partial p as
// round(p * 2^24) + 2^46 (in [0, 2^47) for |p| < 2^22) together with 1 in the count field
// (bits 58-63), by one agent-scope atomic. Integer sums do not depend on the order of arrival,
// so results are deterministic; 32 slices stay below 2^52. The atomic's return value tells the
// last slice that it is last and holds the whole sum; that slice re-zeroes the word. One round
// trip to the coherence point per slice.
//
// A partial the fixed point cannot hold (NaN, +-Inf or |p| >= 2^22) takes an exact escape: its
// slice stores p as fp32 in the slice's side slot of the output, sets the slice's bit in the
// output's mask word (a zeroed 32-bit word) and adds 0 to the sum with 1 in the escape field
// (bits 52-57), releasing the two stores with the add. The last slice, seeing a non-zero escape
// field, acquires them and adds the escaped partials to the fixed-point sum in slice order, so
// NaN and infinities propagate as in an fp32 sum and large values keep fp32 accuracy; it
// re-zeroes the mask. Outputs without an escape pay nothing for it.
constexpr float kFixScale = 16777216.f;
constexpr float kFixLimit = 4194304.f;  // 2^22: partials at or above it (and NaN) escape
constexpr unsigned long long kFixBias = 1ull << 46;
constexpr int kFixEscShift = 52;
constexpr int kFixCountShift = 58;
constexpr int kFixMaxSlices = 32;
// The counter region holds the 64-bit words in its first kFixWordBytes and a 32-bit mask word
// per 64-bit word after them (mask i at byte kFixWordBytes + 4 i).
constexpr size_t kFixWordBytes = 2 << 20;
constexpr size_t kFixMaxWords = kFixWordBytes / 8;

// Where one output's escape goes: its mask word and its slot for slice 0 (slice s at
// side + s * stride).
struct FixEsc {
  uint32_t* mask;
  float* side;
  size_t stride;
};
__device__ __forceinline__ FixEsc fix_esc(unsigned long long* words, size_t i, float* side_base, size_t stride) {
  return {reinterpret_cast<uint32_t*>(reinterpret_cast<char*>(words) + kFixWordBytes) + i, side_base + i, stride};
}

__device__ __forceinline__ bool fix_fits(float p) { return fabsf(p) < kFixLimit; }  // false for NaN

// The word a slice adds for its partial p.
__device__ __forceinline__ unsigned long long fix_word(float p) {
  return fix_fits(p) ? (1ull << kFixCountShift) + (unsigned long long)(__float2ll_rn(p * kFixScale) + (long long)kFixBias)
                     : (1ull << kFixCountShift) + (1ull << kFixEscShift) + kFixBias;
}
// Slice `slice` adds `add` (= fix_word(p)) to word w; returns the word's previous value.
__device__ __forceinline__ unsigned long long fix_issue(unsigned long long* w, unsigned long long add, float p,
                                                        const FixEsc& e, int slice) {
  if (fix_fits(p)) return __hip_atomic_fetch_add(w, add, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  __hip_atomic_store(e.side + (size_t)slice * e.stride, p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  __hip_atomic_fetch_or(e.mask, 1u << slice, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  return __hip_atomic_fetch_add(w, add, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_AGENT);
}
// After the atomic returned `old`: true in the last slice, with the whole sum in *sum, and the
// word (and mask) re-zeroed. Issue every atomic of a lane before finishing any, so their round
// trips overlap.
__device__ __forceinline__ bool fix_finish(unsigned long long* w, unsigned long long old, unsigned long long add,
                                           int slices, const FixEsc& e, float* sum) {
  if ((int)(old >> kFixCountShift) != slices - 1) return false;
  const unsigned long long tot = old + add;
  const long long v = (long long)(tot & ((1ull << kFixEscShift) - 1)) - (long long)slices * (long long)kFixBias;
  float s = (float)v * (1.f / kFixScale);
  if ((tot >> kFixEscShift) & 63ull) {
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
    const uint32_t m = __hip_atomic_load(e.mask, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    for (int i = 0; i < slices; ++i)
      if ((m >> i) & 1u) s += __hip_atomic_load(e.side + (size_t)i * e.stride, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    __hip_atomic_store(e.mask, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
  *sum = s;
  __hip_atomic_store(w, 0ull, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  return true;
}
__device__ __forceinline__ bool fix_add(unsigned long long* w, float p, int slices, int slice, const FixEsc& e,
                                        float* sum) {
  const unsigned long long add = fix_word(p);
  return fix_finish(w, fix_issue(w, add, p, e, slice), add, slices, e, sum);
}

}  // namespace mt
}  // namespace miq
