// Shared device/host helpers for the MI355X (gfx950) quantized-linear library.
#pragma once
#include <hip/hip_runtime.h>
#include <hip/hip_fp16.h>
#include <stdint.h>

#include "../../include/miq.h"

namespace miq {

// ---- error reporting (thread-local message, negative return codes) -------------------
void set_error(const char* fmt, ...);
int fail(int code, const char* fmt, ...);
int check_launch(const char* what);
// MIQ_OK if `bytes` of dynamic LDS fit one workgroup on the current device, else an error.
int require_lds(const char* what, size_t bytes);

#define MIQ_REQUIRE(cond, code, ...)              \
  do {                                            \
    if (!(cond)) return ::miq::fail(code, __VA_ARGS__); \
  } while (0)

inline bool aligned(const void* p, uintptr_t a) { return (reinterpret_cast<uintptr_t>(p) & (a - 1)) == 0; }

// One-row int4 GEMV on the matrix cores (gemv_mma.hip), used by miq_gptq_gemv and by
// miq_gptq_gemv_fused (xmode 1 RMSNorm with norm_w and eps, 2 SwiGLU of a [gate | up] row);
// returns MIQ_ERR_UNSUPPORTED without launching for shapes and modes it does not cover.
int gemv_mma(const void* x, int xd, const int32_t* perm, const int32_t* qw, const int32_t* qz, const void* sc,
             int sd, const float* bias, void* out, int od, int K, int N, int gs, float zoff, void* ws,
             size_t ws_bytes, hipStream_t st, int xmode = 0, const float* norm_w = nullptr, float eps = 0.f);
size_t gemv_mma_workspace(int K, int N);
// Few-row (M <= 16) int4 product on the matrix cores (gemm_small.hip), used by miq_gptq_gemm;
// MIQ_ERR_UNSUPPORTED for shapes it does not cover. xg: gathered copy of x (act-order) or null.
int gemm_small(const __half* x, const __half* xg, const int32_t* qw, const int32_t* qz, const void* sc, int sd,
               const float* bias, void* out, int od, int M, int K, int N, int gs, int bits, float zoff, void* ws,
               size_t ws_bytes, hipStream_t st);
size_t gemm_small_workspace(int M, int K, int N, int gs, int bits, bool perm);  // SIZE_MAX: not covered

// ---- element loads / stores for the activation / output dtypes ---------------------
template <typename T> __device__ __forceinline__ float to_f32(T v);
template <> __device__ __forceinline__ float to_f32<float>(float v) { return v; }
template <> __device__ __forceinline__ float to_f32<__half>(__half v) { return __half2float(v); }

template <typename T> __device__ __forceinline__ T from_f32(float v);
template <> __device__ __forceinline__ float from_f32<float>(float v) { return v; }
template <> __device__ __forceinline__ __half from_f32<__half>(float v) { return __float2half_rn(v); }

// ---- 8 consecutive activations as fp32 (one 16-byte load for fp16, two for fp32) --------
__device__ __forceinline__ void load8(const __half* p, float* v) {
  const uint4 t = *reinterpret_cast<const uint4*>(p);
  const uint32_t w[4] = {t.x, t.y, t.z, t.w};
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    v[2 * i] = __half2float(__ushort_as_half((unsigned short)(w[i] & 0xFFFF)));
    v[2 * i + 1] = __half2float(__ushort_as_half((unsigned short)(w[i] >> 16)));
  }
}
__device__ __forceinline__ void load8(const float* p, float* v) {
  const float4 a = *reinterpret_cast<const float4*>(p);
  const float4 b = *reinterpret_cast<const float4*>(p + 4);
  v[0] = a.x; v[1] = a.y; v[2] = a.z; v[3] = a.w; v[4] = b.x; v[5] = b.y; v[6] = b.z; v[7] = b.w;
}
// two fp32 values (exact fp16 inputs) packed as an fp16 pair
__device__ __forceinline__ uint32_t pack_h2(float a, float b) {
  return (uint32_t)__half_as_ushort(__float2half_rn(a)) | ((uint32_t)__half_as_ushort(__float2half_rn(b)) << 16);
}

// 8 consecutive activations (one int4 packed row, or two int8 rows) as fp16 in the pair order
// that the code unpack produces: int4 (x0,x4) (x1,x5) (x2,x6) (x3,x7); int8, per 4-row word,
// (x0,x2) (x1,x3). A dot product over a packed row is the same sum in that order.
template <int BITS> __device__ __forceinline__ uint4 pack8_pairs(const float* v) {
  if constexpr (BITS == 4)
    return make_uint4(pack_h2(v[0], v[4]), pack_h2(v[1], v[5]), pack_h2(v[2], v[6]), pack_h2(v[3], v[7]));
  else
    return make_uint4(pack_h2(v[0], v[2]), pack_h2(v[1], v[3]), pack_h2(v[4], v[6]), pack_h2(v[5], v[7]));
}

// ---- wavefront (64 lanes) reductions --------------------------------------------------
// Within each row of 16 lanes by DPP moves (quad_perm [1,0,3,2], [2,3,0,1], row_half_mirror,
// row_mirror: every lane ends with its row's total), then the four row totals by v_readlane,
// summed in a fixed order. No LDS round trip (a shuffle across rows is a ds_bpermute each).
// Call with all 64 lanes active; every lane gets the same result.
template <int CTRL> __device__ __forceinline__ float dpp_move(float v) {
  return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, 0xF, 0xF, false));
}
__device__ __forceinline__ float lane_at(float v, int l) {
  return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), l));
}
// Sum over each quad of 4 consecutive lanes (all four active): the pairing of xor 1 then xor 2.
__device__ __forceinline__ float quad_sum(float v) {
  v += dpp_move<0xB1>(v);
  return v + dpp_move<0x4E>(v);
}
__device__ __forceinline__ float wave_sum(float v) {
  v += dpp_move<0xB1>(v);
  v += dpp_move<0x4E>(v);
  v += dpp_move<0x141>(v);
  v += dpp_move<0x140>(v);
  return (lane_at(v, 0) + lane_at(v, 16)) + (lane_at(v, 32) + lane_at(v, 48));
}
__device__ __forceinline__ float wave_max(float v) {
  v = fmaxf(v, dpp_move<0xB1>(v));
  v = fmaxf(v, dpp_move<0x4E>(v));
  v = fmaxf(v, dpp_move<0x141>(v));
  v = fmaxf(v, dpp_move<0x140>(v));
  return fmaxf(fmaxf(lane_at(v, 0), lane_at(v, 16)), fmaxf(lane_at(v, 32), lane_at(v, 48)));
}

// ---- fp16 pairs: 4-bit codes to exact fp16 without a conversion per value ---------------
// OR-ing a code c into the low mantissa bits of 1024.0 (0x6400) gives 1024 + c (or 1024 + 16c
// for a code in bits 4..7) exactly; one packed subtract / fma recovers c. v_dot2 then takes
// two products per instruction with fp32 accumulation.
typedef _Float16 half2v __attribute__((ext_vector_type(2)));

__device__ __forceinline__ half2v as_h2(uint32_t u) { return __builtin_bit_cast(half2v, u); }
// A constant as a register value the compiler cannot see through. The empty asm emits no
// instruction and has no side effects, so the compiler still hoists and shares it like any
// other value; the constant then stays in a register across a loop.
__device__ __forceinline__ uint32_t opaque(uint32_t v) {
  asm("" : "+v"(v));
  return v;
}
// (a & m) | o as one v_and_or_b32 with register operands (with literal m and o the compiler
// splits it in two instructions, each carrying a literal). Plain C++, so that the compiler's
// hazard tracking covers the result where it feeds a matrix-core instruction: it neither pads
// an inline-asm VALU write before an MFMA that reads it nor delays an inline-asm write of a
// register that an issued MFMA is still reading.
__device__ __forceinline__ uint32_t and_or(uint32_t a, uint32_t m, uint32_t o) { return (a & opaque(m)) | opaque(o); }
// codes in bits 0-3 and 16-19 of w
__device__ __forceinline__ half2v nib_lo(uint32_t w) {
  return as_h2(and_or(w, 0x000F000Fu, 0x64006400u)) - (half2v){(_Float16)1024, (_Float16)1024};
}
// codes in bits 4-7 and 20-23 of w
__device__ __forceinline__ half2v nib_hi(uint32_t w) {
  return __builtin_elementwise_fma(as_h2(and_or(w, 0x00F000F0u, 0x64006400u)),
                                   (half2v){(_Float16)0.0625f, (_Float16)0.0625f},
                                   (half2v){(_Float16)-64, (_Float16)-64});
}
// bytes 0 and 2 of w (8-bit codes, 1024 + c is exact for c < 1024)
__device__ __forceinline__ half2v byte02(uint32_t w) {
  return as_h2(and_or(w, 0x00FF00FFu, 0x64006400u)) - (half2v){(_Float16)1024, (_Float16)1024};
}
__device__ __forceinline__ float dot2(half2v a, half2v b, float c) { return __builtin_amdgcn_fdot2(a, b, c, false); }

// Raw scale words of 4 adjacent columns (fp16: 8 bytes, fp32: 16 bytes); converted only when
// used, so that issuing a batch's loads never waits for them.
template <typename ST> __device__ __forceinline__ uint4 load_scales4(const ST* p);
template <> __device__ __forceinline__ uint4 load_scales4<float>(const float* p) {
  return *reinterpret_cast<const uint4*>(p);
}
template <> __device__ __forceinline__ uint4 load_scales4<__half>(const __half* p) {
  const uint2 t = *reinterpret_cast<const uint2*>(p);
  return make_uint4(t.x, t.y, 0u, 0u);
}
template <typename ST> __device__ __forceinline__ void scales4(uint4 r, float* v);
template <> __device__ __forceinline__ void scales4<float>(uint4 r, float* v) {
  v[0] = __uint_as_float(r.x); v[1] = __uint_as_float(r.y); v[2] = __uint_as_float(r.z); v[3] = __uint_as_float(r.w);
}
template <> __device__ __forceinline__ void scales4<__half>(uint4 r, float* v) {
  v[0] = __half2float(__ushort_as_half((unsigned short)(r.x & 0xFFFF)));
  v[1] = __half2float(__ushort_as_half((unsigned short)(r.x >> 16)));
  v[2] = __half2float(__ushort_as_half((unsigned short)(r.y & 0xFFFF)));
  v[3] = __half2float(__ushort_as_half((unsigned short)(r.y >> 16)));
}

// ---- matrix-core operands (v_mfma_f32_16x16x32_f16) --------------------------------------
typedef _Float16 half8v __attribute__((ext_vector_type(8)));
typedef float float4v __attribute__((ext_vector_type(4)));

__device__ __forceinline__ half8v cat4(half2v a, half2v b, half2v c, half2v d) {
  return (half8v){a.x, a.y, b.x, b.y, c.x, c.y, d.x, d.y};
}

// Zero points of 4 adjacent columns (packed codes zw, column s in bits s*BITS) folded into the
// fp16 conversion: zl = 1024 + z + zoff (subtracted from 1024 + q), zh = -(64 + z + zoff).
template <int BITS>
__device__ __forceinline__ void zero_pairs(uint32_t zw, float zoff, half2v* zl, half2v* zh) {
#pragma unroll
  for (int s = 0; s < 4; ++s) {
    const float zf = (float)((zw >> (s * BITS)) & ((1u << BITS) - 1u)) + zoff;
    const _Float16 l = (_Float16)(1024.f + zf), h = (_Float16)(64.f + zf);
    zl[s] = (half2v){l, l};
    zh[s] = (half2v){(_Float16)-h, (_Float16)-h};
  }
}

// MFMA B operand for column s of a lane's 4 columns: the 8 exact integers q - (z + zoff) of one
// 32-wide k step, in the order c0 c4 c1 c5 c2 c6 c3 c7 (int4: one packed word, w[0]) or
// c0 c2 c1 c3 c4 c6 c5 c7 (int8: two words, w[0] and w[1]).
template <int BITS>
__device__ __forceinline__ half8v b_fragment(const uint4* w, int s, half2v zl, half2v zh) {
  const uint32_t w0 = (&w[0].x)[s];
  if constexpr (BITS == 4) {
    const uint32_t w8 = w0 >> 8;
    const half2v h16 = (half2v){(_Float16)0.0625f, (_Float16)0.0625f};
    return cat4(as_h2(and_or(w0, 0x000F000Fu, 0x64006400u)) - zl,
                __builtin_elementwise_fma(as_h2(and_or(w0, 0x00F000F0u, 0x64006400u)), h16, zh),
                as_h2(and_or(w8, 0x000F000Fu, 0x64006400u)) - zl,
                __builtin_elementwise_fma(as_h2(and_or(w8, 0x00F000F0u, 0x64006400u)), h16, zh));
  } else {
    const uint32_t w1 = (&w[1].x)[s];
    return cat4(as_h2(and_or(w0, 0x00FF00FFu, 0x64006400u)) - zl, as_h2(and_or(w0 >> 8, 0x00FF00FFu, 0x64006400u)) - zl,
                as_h2(and_or(w1, 0x00FF00FFu, 0x64006400u)) - zl, as_h2(and_or(w1 >> 8, 0x00FF00FFu, 0x64006400u)) - zl);
  }
}

// ---- LDS DMA: each of the 64 lanes copies 16 (or 4) bytes from its own global address to LDS
// at m0 + 16 * lane (4 * lane). Written as inline asm so that the compiler does not track it:
// the caller waits for these loads itself (s_waitcnt vmcnt) and orders them with a barrier.
typedef __attribute__((address_space(3))) const char lds_cchar;
__device__ __forceinline__ uint32_t lds_addr(const void* p) { return (uint32_t)(uintptr_t)(lds_cchar*)p; }
__device__ __forceinline__ void dma16(const void* g, uint32_t lds) {
  asm volatile("global_load_lds_dwordx4 %0, off" ::"v"(g), "{m0}"(lds) : "memory");
}
__device__ __forceinline__ void dma4(const void* g, uint32_t lds) {
  asm volatile("global_load_lds_dword %0, off" ::"v"(g), "{m0}"(lds) : "memory");
}
// s_waitcnt vmcnt(N) alone (expcnt and lgkmcnt left at their maxima)
template <int N> __device__ __forceinline__ void wait_vmcnt() {
  static_assert(N >= 0 && N < 64, "vmcnt is 6 bits");
  __builtin_amdgcn_s_waitcnt((N & 15) | (7 << 4) | (15 << 8) | ((N >> 4) << 14));
}

// ---- loads through pointers of unknown address space --------------------------------------
// A pointer read from memory (a layer table entry, say) is generic to the compiler, and a
// generic access is a flat instruction, which counts in lgkmcnt as well as vmcnt: every later
// wait for LDS (each barrier waits for lgkmcnt 0) would then also wait for that global load's
// round trip. These helpers load through a global (address space 1) pointer instead; the
// 16- and 8-byte forms go through native vector types, which keep the address space.
#define MIQ_GLOBAL __attribute__((address_space(1)))
typedef uint32_t miq_u32x2 __attribute__((ext_vector_type(2)));
typedef uint32_t miq_u32x4 __attribute__((ext_vector_type(4)));
template <typename T> __device__ __forceinline__ T ldg(const T* p) { return *(const MIQ_GLOBAL T*)p; }
__device__ __forceinline__ uint4 ldg4(const void* p) {
  const miq_u32x4 v = *(const MIQ_GLOBAL miq_u32x4*)p;
  return make_uint4(v.x, v.y, v.z, v.w);
}
__device__ __forceinline__ float4 ldgf4(const void* p) {
  const miq_u32x4 v = *(const MIQ_GLOBAL miq_u32x4*)p;
  return make_float4(__uint_as_float(v.x), __uint_as_float(v.y), __uint_as_float(v.z), __uint_as_float(v.w));
}
__device__ __forceinline__ uint2 ldg2(const void* p) {
  const miq_u32x2 v = *(const MIQ_GLOBAL miq_u32x2*)p;
  return make_uint2(v.x, v.y);
}
template <typename T> __device__ __forceinline__ void stg(T* p, T v) { *(MIQ_GLOBAL T*)p = v; }

// Uniform (scalar) copy of a value that is the same in every lane.
__device__ __forceinline__ int uniform(int v) { return __builtin_amdgcn_readfirstlane(v); }

// Number of workgroups worth launching to cover the whole chip several times over.
constexpr int kCUs = 256;

// Split-K workspaces: every kernel keeps its arrival counters in the same fixed region at the
// start of the workspace (so one call's partial sums can never land on another call's
// counters) and its partials after it. The region is 4 MiB: 64-bit fixed-point words (or int
// counters) in the first 2 MiB, the words' 32-bit escape masks in the next 1 MiB
// (mma_tile.h), 1 MiB unused.
constexpr size_t kCounterBytes = 4 << 20;
constexpr int kMaxCounters = (int)((2 << 20) / 4);

}  // namespace miq
