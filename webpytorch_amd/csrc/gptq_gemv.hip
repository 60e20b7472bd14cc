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
#include <algorithm>
#include <mutex>
#include <type_traits>

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
// Decode GEMV / skinny GEMM: out[M][N] = x[M][K] @ W + bias, MR rows of x per workgroup.
//
// Grid (tiles, ksplit, ceil(M / MR)), W waves per workgroup. A wave covers 256 columns: a lane
// owns 4 adjacent columns and reads them with one 16-byte load per packed row, so a wave reads
// 1 KB contiguous per row. The K dimension is cut into batches of RPW packed rows (BK = RPW *
// per activations; BK divides gs, so a batch lies in one group). A workgroup takes W
// consecutive batches of its column tile, one per wave (with no workspace, a wave loops over
// every W-th batch of the whole K range). Latency is hidden by occupancy: every wave issues
// its whole batch (RPW 16-byte loads per lane) at once, before the workgroup stages x.
// Per batch and column: part = sum_k x_k q_k, acc += s * (part - (z + zoff) * sum_k x_k).
// fp16 activations take the v_dot2 path (codes converted to exact fp16 pairs); fp32
// activations take an fp32 FMA path. The waves are summed in a fixed order through LDS.
// With ksplit > 1 the workgroups of one column tile store fp32 partials in the workspace;
// the last to arrive (device-scope atomic counter) sums them in ksplit order, adds the bias,
// writes the output and re-arms the counter to zero, so results are deterministic.

constexpr size_t kGemvMmaMinBytes = 0;  // int4 codes of a layer from which one row takes gemv_mma (every size)
constexpr int kGemvMinWgs = 1;          // split K further while fewer workgroups than this would run
constexpr int kGemvMaxWaves = 16;       // waves per workgroup (1024 threads)
constexpr int kGemvSplitWaves = 4;      // waves per workgroup when K is split across workgroups
constexpr int kGemvStageBytes = 64 * 1024;  // LDS for the staged activations (no workspace)

template <int BITS> struct Codes;

// int4: one word = 8 consecutive rows of one column, row j in bits 4j..4j+3.
template <> struct Codes<4> {
  static constexpr int PER = 8, PAIRS = 4;
  // the codes as fp16 pairs (c0,c4) (c1,c5) (c2,c6) (c3,c7)
  __device__ __forceinline__ static void pairs(uint32_t w, half2v* p) {
    const uint32_t w8 = w >> 8;
    p[0] = nib_lo(w);
    p[1] = nib_hi(w);
    p[2] = nib_lo(w8);
    p[3] = nib_hi(w8);
  }
  __device__ __forceinline__ static float dotf(uint32_t w, const float* x, float part) {
    const uint32_t lo = w & 0x0F0F0F0Fu;         // rows 0,2,4,6
    const uint32_t hi = (w >> 4) & 0x0F0F0F0Fu;  // rows 1,3,5,7
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

// int8: one word = 4 consecutive rows of one column, row j in bits 8j..8j+7.
template <> struct Codes<8> {
  static constexpr int PER = 4, PAIRS = 2;
  // the codes as fp16 pairs (c0,c2) (c1,c3)
  __device__ __forceinline__ static void pairs(uint32_t w, half2v* p) {
    p[0] = byte02(w);
    p[1] = byte02(w >> 8);
  }
  __device__ __forceinline__ static float dotf(uint32_t w, const float* x, float part) {
    part = fmaf(x[0], (float)(w & 0xFFu), part);
    part = fmaf(x[1], (float)((w >> 8) & 0xFFu), part);
    part = fmaf(x[2], (float)((w >> 16) & 0xFFu), part);
    part = fmaf(x[3], (float)(w >> 24), part);
    return part;
  }
};

template <int RPW> struct GemvBatch {
  uint4 w[RPW];
  uint4 s;     // raw scale words
  uint32_t z;  // raw packed zero word (shifted to this lane's columns when used)
};

// Input transforms applied while staging x (XMODE): none; RMSNorm of each row of x with
// weight norm_w (x / sqrt(mean(x^2) + eps) * w, every workgroup recomputes the row's mean
// square); SwiGLU of a [gate | up] row of 2K values (silu(gate) * up).
template <int BITS, int MR, int RPW, typename XT, typename ST, typename OT, int XMODE>
__global__ __launch_bounds__(64 * kGemvMaxWaves) void gptq_gemv_kernel(
    const XT* __restrict__ x, const int32_t* __restrict__ perm, const uint32_t* __restrict__ qw,
    const uint32_t* __restrict__ qz, const ST* __restrict__ sc, const float* bias, OT* out,
    float* __restrict__ ws, int* __restrict__ counters, int M, int K, int N, int gs, float zoff, int rows_per_wg,
    int ksplit, const float* __restrict__ norm_w, float eps) {
  using C = Codes<BITS>;
  constexpr int PER = C::PER, PAIRS = C::PAIRS;
  constexpr int BK = RPW * PER;
  constexpr bool kHalf = std::is_same<XT, __half>::value;
  constexpr int XB = kHalf ? 2 : 4;
  constexpr uint32_t MASK = (1u << BITS) - 1u;
  extern __shared__ __align__(16) unsigned char lds_raw[];
  __shared__ int is_last;
  __shared__ float ss_red[kGemvMaxWaves][MR];

  const int W = blockDim.x >> 6;
  const int lane = threadIdx.x & 63;
  const int wave = uniform(threadIdx.x >> 6);
  const int tile = blockIdx.x, ks = blockIdx.y, m0 = blockIdx.z * MR;
  const int r0 = ks * rows_per_wg;
  const int r1 = min(K / PER, r0 + rows_per_wg);
  const int L = (r1 - r0) * PER;   // staged activations per row of x (a multiple of BK)
  const int nb = (r1 - r0) / RPW;  // batches in this workgroup
  const int n0 = tile * 256 + lane * 4;
  const bool colok = n0 < N;
  const int NZ = N / PER;
  const int zshift = (n0 % PER) * BITS;

  auto load_batch = [&](int b, GemvBatch<RPW>& B) {
    const int rb = r0 + b * RPW;
    const uint32_t* base = qw + (size_t)rb * N + n0;
#pragma unroll
    for (int r = 0; r < RPW; ++r) B.w[r] = *reinterpret_cast<const uint4*>(base + (size_t)r * N);
    const int g = rb * PER / gs;
    B.s = load_scales4<ST>(sc + (size_t)g * N + n0);
    B.z = qz[(size_t)g * NZ + n0 / PER];
  };

  // ---- a wave's first two batches of weights, issued before the activations are staged ----
  GemvBatch<RPW> B, B2;
  const int b = wave;
  const bool has1 = colok && b < nb, has2 = colok && b + W < nb;
  if (has1) load_batch(b, B);
  if (has2) load_batch(b + W, B2);

  // ---- RMSNorm: mean square of every row of x over the full K ----
  const int xstride = XMODE == 2 ? 2 * K : K;
  float inv_r[MR];
  if constexpr (XMODE == 1) {
#pragma unroll
    for (int m = 0; m < MR; ++m) {
      float ss = 0.f;
      if (m0 + m < M)
        for (int i = threadIdx.x; i < K; i += blockDim.x) {
          const float v = to_f32(x[(size_t)(m0 + m) * K + i]);
          ss += v * v;
        }
      ss = wave_sum(ss);
      if (lane == 0) ss_red[wave][m] = ss;
    }
    __syncthreads();
#pragma unroll
    for (int m = 0; m < MR; ++m) {
      float t = 0.f;
      for (int w = 0; w < W; ++w) t += ss_red[w][m];
      inv_r[m] = sqrtf(t / (float)K + eps);
    }
  }

  // ---- stage x (through perm and the input transform) in LDS and the per-batch sums of x ----
  _Float16* xs_h = reinterpret_cast<_Float16*>(lds_raw);
  float* xs_f = reinterpret_cast<float*>(lds_raw);
  const size_t xs_bytes = ((size_t)MR * L * XB + 15) & ~(size_t)15;
  float* xsum = reinterpret_cast<float*>(lds_raw + xs_bytes);
  // 8 consecutive activations per thread and step (one int4 packed row, two int8 rows)
  constexpr int SEG = BK / 8;  // threads per batch
  const int cpr = L / 8;       // chunks per row of x
  for (int ci = threadIdx.x; ci < MR * cpr; ci += blockDim.x) {
    const int m = ci / cpr, kk = (ci - m * cpr) * 8;
    const int k = r0 * PER + kk;
    float v[8];
    if (m0 + m < M) {
      const XT* xr = x + (size_t)(m0 + m) * xstride;
      int idx[8];
#pragma unroll
      for (int j = 0; j < 8; ++j) idx[j] = perm ? perm[k + j] : k + j;
      if (perm) {
#pragma unroll
        for (int j = 0; j < 8; ++j) v[j] = to_f32(xr[idx[j]]);
      } else {
        load8(xr + k, v);
      }
      if constexpr (XMODE == 1) {
#pragma unroll
        for (int j = 0; j < 8; ++j) v[j] = (v[j] / inv_r[m]) * norm_w[idx[j]];
      } else if constexpr (XMODE == 2) {
        float u[8];
        if (perm) {
#pragma unroll
          for (int j = 0; j < 8; ++j) u[j] = to_f32(xr[K + idx[j]]);
        } else {
          load8(xr + K + k, u);
        }
#pragma unroll
        for (int j = 0; j < 8; ++j) v[j] = (v[j] * (1.f / (1.f + expf(-v[j])))) * u[j];
      }
    } else {
#pragma unroll
      for (int j = 0; j < 8; ++j) v[j] = 0.f;
    }
    // every aligned run of SEG threads is one batch of one row of x, all of them present
    float sum = ((v[0] + v[1]) + (v[2] + v[3])) + ((v[4] + v[5]) + (v[6] + v[7]));
#pragma unroll
    for (int o = 1; o < SEG; o <<= 1) sum += __shfl_xor(sum, o, 64);
    if ((lane & (SEG - 1)) == 0) xsum[m * nb + kk / BK] = sum;
    if constexpr (kHalf) {
      *reinterpret_cast<uint4*>(xs_h + (size_t)m * L + kk) = pack8_pairs<BITS>(v);
    } else {
      float4* d = reinterpret_cast<float4*>(xs_f + (size_t)m * L + kk);
      d[0] = make_float4(v[0], v[1], v[2], v[3]);
      d[1] = make_float4(v[4], v[5], v[6], v[7]);
    }
  }
  __syncthreads();

  float acc[MR][4];
#pragma unroll
  for (int m = 0; m < MR; ++m)
#pragma unroll
    for (int c = 0; c < 4; ++c) acc[m][c] = 0.f;

  auto compute = [&](int bb, const GemvBatch<RPW>& B) {
    float part[MR][4];
#pragma unroll
    for (int m = 0; m < MR; ++m)
#pragma unroll
      for (int c = 0; c < 4; ++c) part[m][c] = 0.f;
#pragma unroll
    for (int r = 0; r < RPW; ++r) {
      uint32_t wv[4] = {B.w[r].x, B.w[r].y, B.w[r].z, B.w[r].w};
      // An empty asm that takes this row's words and the running sums keeps the rows in order:
      // the compiler would otherwise unpack every row of the batch at once (4x the registers)
      // and spill.
      asm volatile("" : "+v"(wv[0]), "+v"(wv[1]), "+v"(wv[2]), "+v"(wv[3]), "+v"(part[0][0]), "+v"(part[0][1]),
                   "+v"(part[0][2]), "+v"(part[0][3]));
      const int row = bb * RPW + r;  // local packed row
      if constexpr (kHalf) {
        half2v p[4][PAIRS];
#pragma unroll
        for (int c = 0; c < 4; ++c) C::pairs(wv[c], p[c]);
#pragma unroll
        for (int m = 0; m < MR; ++m) {
          const half2v* xp = reinterpret_cast<const half2v*>(xs_h + (size_t)m * L + row * PER);
          half2v xv[PAIRS];
#pragma unroll
          for (int i = 0; i < PAIRS; ++i) xv[i] = xp[i];
#pragma unroll
          for (int c = 0; c < 4; ++c)
#pragma unroll
            for (int i = 0; i < PAIRS; ++i) part[m][c] = dot2(xv[i], p[c][i], part[m][c]);
        }
      } else {
#pragma unroll
        for (int m = 0; m < MR; ++m) {
          const float* xp = xs_f + (size_t)m * L + row * PER;
          float xv[PER];
#pragma unroll
          for (int j = 0; j < PER; j += 4) {
            const float4 t = *reinterpret_cast<const float4*>(xp + j);
            xv[j] = t.x; xv[j + 1] = t.y; xv[j + 2] = t.z; xv[j + 3] = t.w;
          }
#pragma unroll
          for (int c = 0; c < 4; ++c) part[m][c] = C::dotf(wv[c], xv, part[m][c]);
        }
      }
    }
    float zf[4], sf[4];
    scales4<ST>(B.s, sf);
    const uint32_t zw = B.z >> zshift;
#pragma unroll
    for (int c = 0; c < 4; ++c) zf[c] = (float)((zw >> (c * BITS)) & MASK) + zoff;
#pragma unroll
    for (int m = 0; m < MR; ++m) {
      const float xb = xsum[m * nb + bb];
#pragma unroll
      for (int c = 0; c < 4; ++c) acc[m][c] = fmaf(sf[c], fmaf(-zf[c], xb, part[m][c]), acc[m][c]);
    }
  };

  // straight-line code keeps both batches in flight (a loop makes the compiler wait on the
  // prefetched one); further batches, if any, go one at a time
  if (has1) compute(b, B);
  if (has2) compute(b + W, B2);
  for (int bb = b + 2 * W; colok && bb < nb; bb += W) {
    load_batch(bb, B);
    compute(bb, B);
  }

  // ---- fixed-order reduction of the W waves ----
  const size_t stage = xs_bytes + (((size_t)MR * nb * 4 + 15) & ~(size_t)15);
  float* red = reinterpret_cast<float*>(lds_raw + stage);  // [W][MR][256]
#pragma unroll
  for (int m = 0; m < MR; ++m)
#pragma unroll
    for (int c = 0; c < 4; ++c) red[(wave * MR + m) * 256 + lane * 4 + c] = acc[m][c];
  __syncthreads();

  if (ksplit == 1) {
    for (int i = threadIdx.x; i < MR * 256; i += blockDim.x) {
      const int m = i >> 8, q = i & 255, n = tile * 256 + q;
      if (m0 + m >= M || n >= N) continue;
      float s = 0.f;
      for (int w = 0; w < W; ++w) s += red[(w * MR + m) * 256 + q];
      if (bias) s += bias[n];
      out[(size_t)(m0 + m) * N + n] = from_f32<OT>(s);
    }
    return;
  }

  // Partials are exchanged with device-scope (agent) atomic stores and loads, which bypass
  // the per-XCD L2, so no cache-wide writeback or invalidate is needed: each thread waits for
  // its stores to complete before the workgroup counts itself in, and the last workgroup reads
  // the partials with device-scope loads after it has seen the final count.
  for (int i = threadIdx.x; i < MR * 256; i += blockDim.x) {
    const int m = i >> 8, q = i & 255, n = tile * 256 + q;
    if (m0 + m >= M || n >= N) continue;
    float s = 0.f;
    for (int w = 0; w < W; ++w) s += red[(w * MR + m) * 256 + q];
    __hip_atomic_store(ws + ((size_t)ks * M + m0 + m) * N + n, s, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
  int* ctr = counters + (size_t)blockIdx.z * gridDim.x + tile;
  if (threadIdx.x == 0)
    is_last = __hip_atomic_fetch_add(ctr, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == ksplit - 1;
  __syncthreads();
  if (!is_last) return;
  for (int i = threadIdx.x; i < MR * 256; i += blockDim.x) {
    const int m = i >> 8, q = i & 255, n = tile * 256 + q;
    if (m0 + m >= M || n >= N) continue;
    // issue the partial loads four at a time; the sum stays in ksplit order
    const float* pp = ws + (size_t)(m0 + m) * N + n;
    const size_t stride = (size_t)M * N;
    float s = 0.f;
    int k2 = 0;
    for (; k2 + 4 <= ksplit; k2 += 4) {
      const float a0 = __hip_atomic_load(pp + (k2 + 0) * stride, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      const float a1 = __hip_atomic_load(pp + (k2 + 1) * stride, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      const float a2 = __hip_atomic_load(pp + (k2 + 2) * stride, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      const float a3 = __hip_atomic_load(pp + (k2 + 3) * stride, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      s = (((s + a0) + a1) + a2) + a3;
    }
    for (; k2 < ksplit; ++k2) s += __hip_atomic_load(pp + k2 * stride, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    if (bias) s += bias[n];
    out[(size_t)(m0 + m) * N + n] = from_f32<OT>(s);
  }
  if (threadIdx.x == 0) __hip_atomic_store(ctr, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);  // re-armed
}

// Launch geometry shared by the workspace query and the launch.
struct GemvPlan {
  int mr, rpw, waves, tiles, mblocks, ksplit, rows_per_wg;
  size_t lds, counter_bytes, ws_bytes;
};

static int gemv_plan(int M, int K, int N, int gs, int bits, int x_dtype, bool have_ws, GemvPlan* p) {
  const int per = 32 / bits;
  int rpw = 0;
  for (int r = 8; r >= 4; r >>= 1)
    if (gs % (r * per) == 0) { rpw = r; break; }
  MIQ_REQUIRE(rpw, MIQ_ERR_UNSUPPORTED, "gptq_gemv: group size %d (needs a multiple of %d)", gs, 4 * per);
  p->rpw = rpw;
  p->mr = M >= 8 ? 8 : (M >= 4 ? 4 : 1);
  p->tiles = (N + 255) / 256;
  p->mblocks = (M + p->mr - 1) / p->mr;
  const int xb = x_dtype == MIQ_F16 ? 2 : 4;
  const int nbt = K / per / rpw;  // batches per column tile
  const int wmax = kGemvSplitWaves;
  const int base = p->tiles * p->mblocks;
  int waves, ksplit;
  // wide layers fill the chip by columns alone: no K split, each wave streams several batches
  const bool wide = base >= 2 * kCUs && (size_t)p->mr * K * xb <= (size_t)kGemvStageBytes;
  if (have_ws && base <= kMaxCounters && !wide) {
    // one batch per wave; fewer waves per workgroup while too few workgroups would run
    waves = nbt < wmax ? nbt : wmax;
    ksplit = (nbt + waves - 1) / waves;
    while (waves > 1 && base * ksplit < kGemvMinWgs) {
      waves = (waves + 1) / 2;
      ksplit = (nbt + waves - 1) / waves;
    }
  } else {
    // every wave takes two batches (both in flight at once): ceil(batches / 2) waves
    waves = (nbt + 1) / 2;
    waves = waves > kGemvMaxWaves ? kGemvMaxWaves : waves;
    ksplit = 1;
    MIQ_REQUIRE((size_t)p->mr * K * xb <= (size_t)kGemvStageBytes, MIQ_ERR_INVALID,
                "gptq_gemv: K=%d needs a workspace (see miq_gptq_gemv_workspace)", K);
  }
  const int rows_per_wg = ksplit == 1 ? K / per : waves * rpw;
  p->waves = waves;
  p->ksplit = ksplit;
  p->rows_per_wg = rows_per_wg;
  const int L = rows_per_wg * per, nb = rows_per_wg / rpw;
  p->lds = (((size_t)p->mr * L * xb + 15) & ~(size_t)15) + (((size_t)p->mr * nb * 4 + 15) & ~(size_t)15) +
           (size_t)waves * p->mr * 256 * 4;
  p->counter_bytes = ksplit > 1 ? kCounterBytes : 0;
  p->ws_bytes = ksplit > 1 ? p->counter_bytes + (size_t)ksplit * M * N * 4 : 0;
  return MIQ_OK;
}

template <int BITS, int MR, int RPW, typename XT, typename ST, typename OT, int XMODE>
static int launch_gemv(const GemvPlan& p, const void* x, const int32_t* perm, const int32_t* qw,
                       const int32_t* qz, const void* sc, const float* bias, void* out, void* ws,
                       int M, int K, int N, int gs, float zoff, const float* norm_w, float eps, hipStream_t st) {
  auto kern = gptq_gemv_kernel<BITS, MR, RPW, XT, ST, OT, XMODE>;
  int* counters = p.ksplit > 1 ? static_cast<int*>(ws) : nullptr;
  float* partials = p.ksplit > 1 ? reinterpret_cast<float*>(static_cast<char*>(ws) + p.counter_bytes) : nullptr;
  if (p.lds > 64 * 1024) {
    const int rc = require_lds("gptq_gemv", p.lds);
    if (rc) return rc;
  }
  dim3 grid(p.tiles, p.ksplit, p.mblocks);
  hipLaunchKernelGGL(kern, grid, dim3(64 * p.waves), p.lds, st, static_cast<const XT*>(x), perm,
                     reinterpret_cast<const uint32_t*>(qw), reinterpret_cast<const uint32_t*>(qz),
                     static_cast<const ST*>(sc), bias, static_cast<OT*>(out), partials, counters, M, K, N,
                     gs, zoff, p.rows_per_wg, p.ksplit, norm_w, eps);
  return check_launch("gptq_gemv");
}

template <int BITS, int MR, int RPW>
static int gemv_types(const GemvPlan& p, const void* x, int xd, const int32_t* perm, const int32_t* qw,
                      const int32_t* qz, const void* sc, int sd, const float* bias, void* out, int od,
                      void* ws, int M, int K, int N, int gs, float zoff, hipStream_t st) {
#define MIQ_GEMV_CASE(XT, ST, OT) \
  return launch_gemv<BITS, MR, RPW, XT, ST, OT, 0>(p, x, perm, qw, qz, sc, bias, out, ws, M, K, N, gs, zoff, nullptr, 0.f, st)
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

template <int BITS>
static int gemv_dispatch(const GemvPlan& p, const void* x, int xd, const int32_t* perm, const int32_t* qw,
                         const int32_t* qz, const void* sc, int sd, const float* bias, void* out, int od,
                         void* ws, int M, int K, int N, int gs, float zoff, hipStream_t st) {
#define MIQ_GEMV_MR(MR, RPW) \
  if (p.mr == MR && p.rpw == RPW) \
    return gemv_types<BITS, MR, RPW>(p, x, xd, perm, qw, qz, sc, sd, bias, out, od, ws, M, K, N, gs, zoff, st)
  MIQ_GEMV_MR(1, 8); MIQ_GEMV_MR(4, 8); MIQ_GEMV_MR(8, 8);
  MIQ_GEMV_MR(1, 4); MIQ_GEMV_MR(4, 4); MIQ_GEMV_MR(8, 4);
#undef MIQ_GEMV_MR
  return fail(MIQ_ERR_UNSUPPORTED, "gptq_gemv: no kernel for mr=%d rpw=%d", p.mr, p.rpw);
}

// Fused-input decode GEMV: one row of fp32 activations, fp32 output, int4, RMSNorm (XMODE 1) or
// SwiGLU (XMODE 2) applied while staging.
template <int XMODE>
static int gemv_fused_dispatch(const GemvPlan& p, const void* x, const int32_t* perm, const int32_t* qw,
                               const int32_t* qz, const void* sc, int sd, const float* bias, void* out, void* ws,
                               int M, int K, int N, int gs, int bits, float zoff, const float* norm_w, float eps,
                               hipStream_t st) {
  MIQ_REQUIRE(p.mr == 1, MIQ_ERR_UNSUPPORTED, "gptq_gemv_fused: one row only (M=%d)", M);
#define MIQ_GEMV_FUSED(B, RPW, ST) \
  return launch_gemv<B, 1, RPW, float, ST, float, XMODE>(p, x, perm, qw, qz, sc, bias, out, ws, M, K, N, gs, zoff, norm_w, eps, st)
  if (bits == 4) {
    if (p.rpw == 8) { if (sd == MIQ_F16) MIQ_GEMV_FUSED(4, 8, __half); MIQ_GEMV_FUSED(4, 8, float); }
    if (sd == MIQ_F16) MIQ_GEMV_FUSED(4, 4, __half);
    MIQ_GEMV_FUSED(4, 4, float);
  }
  if (p.rpw == 8) { if (sd == MIQ_F16) MIQ_GEMV_FUSED(8, 8, __half); MIQ_GEMV_FUSED(8, 8, float); }
  if (sd == MIQ_F16) MIQ_GEMV_FUSED(8, 4, __half);
  MIQ_GEMV_FUSED(8, 4, float);
#undef MIQ_GEMV_FUSED
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

static int gemv_check(const char* who, const void* x, int x_dtype, const int32_t* qweight, const int32_t* qzeros,
                      const void* scales, int scales_dtype, void* out, int out_dtype, int M, int K, int N,
                      int gs, int bits) {
  int rc = check_gptq_dims(who, K, N, gs, bits);
  if (rc) return rc;
  MIQ_REQUIRE(M >= 0, MIQ_ERR_INVALID, "%s: M=%d", who, M);
  if (M == 0) return MIQ_OK;
  MIQ_REQUIRE(x && qweight && qzeros && scales && out, MIQ_ERR_INVALID, "%s: null pointer", who);
  MIQ_REQUIRE(N % 4 == 0 && aligned(qweight, 16) && aligned(scales, scales_dtype == MIQ_F16 ? 8 : 16) &&
                  aligned(x, 16) && K % 8 == 0,
              MIQ_ERR_ALIGN, "%s: x and qweight must be 16-byte aligned, N %% 4 == 0 and K %% 8 == 0", who);
  MIQ_REQUIRE(x_dtype == MIQ_F16 || x_dtype == MIQ_F32, MIQ_ERR_UNSUPPORTED, "%s: x dtype", who);
  MIQ_REQUIRE(scales_dtype == MIQ_F16 || scales_dtype == MIQ_F32, MIQ_ERR_UNSUPPORTED, "%s: scales dtype", who);
  MIQ_REQUIRE(out_dtype == MIQ_F16 || out_dtype == MIQ_F32, MIQ_ERR_UNSUPPORTED, "%s: out dtype", who);
  return MIQ_OK;
}

extern "C" int miq_gptq_gemv_workspace(int M, int K, int N, int gs, int bits, int x_dtype, size_t* bytes) {
  MIQ_REQUIRE(bytes, MIQ_ERR_INVALID, "gptq_gemv_workspace: null output");
  *bytes = 0;
  int rc = check_gptq_dims("gptq_gemv_workspace", K, N, gs, bits);
  if (rc) return rc;
  MIQ_REQUIRE(M >= 0, MIQ_ERR_INVALID, "gptq_gemv_workspace: M=%d", M);
  if (M == 0) return MIQ_OK;
  GemvPlan p;
  rc = gemv_plan(M, K, N, gs, bits, x_dtype, true, &p);
  if (rc) return rc;
  *bytes = p.ws_bytes;
  if (M == 1 && bits == 4 && (size_t)K * N / 2 >= kGemvMmaMinBytes)
    *bytes = std::max(*bytes, gemv_mma_workspace(K, N));
  return MIQ_OK;
}

extern "C" int miq_gptq_gemv(const void* x, int x_dtype, const int32_t* perm, const int32_t* qweight,
                             const int32_t* qzeros, const void* scales, int scales_dtype, const float* bias,
                             void* out, int out_dtype, int M, int K, int N, int gs, int bits,
                             float zero_offset, void* workspace, size_t workspace_bytes, void* stream) {
  int rc = gemv_check("gptq_gemv", x, x_dtype, qweight, qzeros, scales, scales_dtype, out, out_dtype, M, K, N,
                      gs, bits);
  if (rc || M == 0) return rc;
  // one row of an int4 layer: the matrix-core GEMV (it declines shapes it does not cover)
  if (M == 1 && bits == 4 && (size_t)K * N / 2 >= kGemvMmaMinBytes &&
      (workspace == nullptr || aligned(workspace, 256))) {
    rc = gemv_mma(x, x_dtype, perm, qweight, qzeros, scales, scales_dtype, bias, out, out_dtype, K, N, gs,
                  zero_offset, workspace, workspace_bytes, static_cast<hipStream_t>(stream));
    if (rc != MIQ_ERR_UNSUPPORTED) return rc;
  }
  GemvPlan p;
  rc = gemv_plan(M, K, N, gs, bits, x_dtype, workspace != nullptr, &p);
  if (rc) return rc;
  if (p.ksplit > 1) {
    MIQ_REQUIRE(workspace_bytes >= p.ws_bytes && aligned(workspace, 256), MIQ_ERR_INVALID,
                "gptq_gemv: workspace of %zu bytes (256-byte aligned) needed, %zu given", p.ws_bytes,
                workspace_bytes);
  }
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (bits == 4)
    return gemv_dispatch<4>(p, x, x_dtype, perm, qweight, qzeros, scales, scales_dtype, bias, out, out_dtype,
                            workspace, M, K, N, gs, zero_offset, st);
  return gemv_dispatch<8>(p, x, x_dtype, perm, qweight, qzeros, scales, scales_dtype, bias, out, out_dtype,
                          workspace, M, K, N, gs, zero_offset, st);
}

extern "C" int miq_gptq_gemv_fused(const float* x, int x_mode, const float* norm_w, float eps, const int32_t* perm,
                                   const int32_t* qweight, const int32_t* qzeros, const void* scales, int scales_dtype,
                                   const float* bias, float* out, int M, int K, int N, int gs, int bits,
                                   float zero_offset, void* workspace, size_t workspace_bytes, void* stream) {
  if (x_mode == MIQ_X_PLAIN)
    return miq_gptq_gemv(x, MIQ_F32, perm, qweight, qzeros, scales, scales_dtype, bias, out, MIQ_F32, M, K, N, gs,
                         bits, zero_offset, workspace, workspace_bytes, stream);
  MIQ_REQUIRE(x_mode == MIQ_X_RMSNORM || x_mode == MIQ_X_SWIGLU, MIQ_ERR_UNSUPPORTED, "gptq_gemv_fused: x_mode %d",
              x_mode);
  MIQ_REQUIRE(x_mode != MIQ_X_RMSNORM || norm_w, MIQ_ERR_INVALID, "gptq_gemv_fused: RMSNorm needs its weight");
  int rc = gemv_check("gptq_gemv_fused", x, MIQ_F32, qweight, qzeros, scales, scales_dtype, out, MIQ_F32, M, K, N, gs,
                      bits);
  if (rc || M == 0) return rc;
  // one row of an int4 layer in k order: the matrix-core GEMV with the transform in its staging
  if (M == 1 && bits == 4 && !perm && (workspace == nullptr || aligned(workspace, 256))) {
    rc = gemv_mma(x, MIQ_F32, nullptr, qweight, qzeros, scales, scales_dtype, bias, out, MIQ_F32, K, N, gs,
                  zero_offset, workspace, workspace_bytes, static_cast<hipStream_t>(stream),
                  x_mode == MIQ_X_RMSNORM ? 1 : 2, norm_w, eps);
    if (rc != MIQ_ERR_UNSUPPORTED) return rc;
  }
  GemvPlan p;
  rc = gemv_plan(M, K, N, gs, bits, MIQ_F32, workspace != nullptr, &p);
  if (rc) return rc;
  if (p.ksplit > 1) {
    MIQ_REQUIRE(workspace_bytes >= p.ws_bytes && aligned(workspace, 256), MIQ_ERR_INVALID,
                "gptq_gemv_fused: workspace of %zu bytes (256-byte aligned) needed, %zu given", p.ws_bytes,
                workspace_bytes);
  }
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (x_mode == MIQ_X_RMSNORM)
    return gemv_fused_dispatch<1>(p, x, perm, qweight, qzeros, scales, scales_dtype, bias, out, workspace, M, K, N, gs,
                                  bits, zero_offset, norm_w, eps, st);
  return gemv_fused_dispatch<2>(p, x, perm, qweight, qzeros, scales, scales_dtype, bias, out, workspace, M, K, N, gs,
                                bits, zero_offset, nullptr, 0.f, st);
}

// ------------------------------------------------------------------------------------
// The GEMV with no workspace argument and no allocation: its split-K workspace is a fixed
// device array of this file. HIP gives every device its own copy of the array; host code
// reaches a device's copy only through the address hipGetSymbolAddress returns while that
// device is current (the array's name in host code is a host-side stand-in, not a device
// address). Each device's address is looked up once, on the first call made on it, which also
// clears the array's counter region with a fill kernel on the caller's stream (the kernels
// leave it zero after every call). That first call must run eagerly: under graph capture the
// clear would only be recorded, so a first call made while the stream captures is refused
// (MIQ_ERR_INVALID) and sets nothing up.
namespace miq {
namespace na {

constexpr size_t kScratchBytes = 16u << 20;  // counter region (4 MiB) + 12 MiB of partials
constexpr int kMaxDevices = 64;

__device__ __align__(256) unsigned char scratch[kScratchBytes];

__global__ __launch_bounds__(256) void zero_words_kernel(uint4* p, size_t n) {
  for (size_t i = (size_t)blockIdx.x * 256 + threadIdx.x; i < n; i += (size_t)gridDim.x * 256)
    p[i] = make_uint4(0u, 0u, 0u, 0u);
}

std::mutex g_lock;
void* g_ptr[kMaxDevices];

// The current device's copy of the scratch array (set up on its first use) in *out; 0 or the
// error code, with the error recorded.
int device_scratch(hipStream_t st, void** out) {
  *out = nullptr;
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess || dev < 0 || dev >= kMaxDevices)
    return fail(MIQ_ERR_HIP, "gptq_gemv_noalloc: hipGetDevice: %s (device %d)", hipGetErrorString(e), dev);
  std::lock_guard<std::mutex> g(g_lock);
  if (!g_ptr[dev]) {
    hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
    e = hipStreamIsCapturing(st, &cs);
    if (e != hipSuccess) return fail(MIQ_ERR_HIP, "gptq_gemv_noalloc: hipStreamIsCapturing: %s", hipGetErrorString(e));
    if (cs != hipStreamCaptureStatusNone)
      return fail(MIQ_ERR_INVALID, "gptq_gemv_noalloc: the first call on a device sets up its scratch array and must "
                                   "run outside graph capture (make one eager call first)");
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !p) return fail(MIQ_ERR_HIP, "gptq_gemv_noalloc: hipGetSymbolAddress: %s", hipGetErrorString(e));
    hipLaunchKernelGGL(zero_words_kernel, dim3(256), dim3(256), 0, st, static_cast<uint4*>(p), kCounterBytes / 16);
    const int rc = check_launch("gptq_gemv_noalloc scratch clear");
    if (rc) return rc;
    g_ptr[dev] = p;
  }
  *out = g_ptr[dev];
  return MIQ_OK;
}

}  // namespace na
}  // namespace miq

extern "C" size_t miq_gptq_gemv_noalloc_max_bytes(void) { return miq::na::kScratchBytes; }

extern "C" int miq_gptq_gemv_noalloc(const void* x, int x_dtype, const int32_t* perm, const int32_t* qweight,
                                     const int32_t* qzeros, const void* scales, int scales_dtype, const float* bias,
                                     void* out, int out_dtype, int M, int K, int N, int gs, int bits,
                                     float zero_offset, void* stream) {
  int rc = gemv_check("gptq_gemv_noalloc", x, x_dtype, qweight, qzeros, scales, scales_dtype, out, out_dtype, M, K,
                      N, gs, bits);
  if (rc || M == 0) return rc;
  size_t need = 0;
  rc = miq_gptq_gemv_workspace(M, K, N, gs, bits, x_dtype, &need);
  if (rc) return rc;
  MIQ_REQUIRE(need <= na::kScratchBytes, MIQ_ERR_INVALID,
              "gptq_gemv_noalloc: M=%d K=%d N=%d needs %zu bytes of split-K workspace, the fixed scratch holds %zu "
              "(use miq_gptq_gemv with a workspace)",
              M, K, N, need, na::kScratchBytes);
  hipStream_t st = static_cast<hipStream_t>(stream);
  void* ws = nullptr;
  rc = na::device_scratch(st, &ws);
  if (rc) return rc;
  return miq_gptq_gemv(x, x_dtype, perm, qweight, qzeros, scales, scales_dtype, bias, out, out_dtype, M, K, N, gs,
                       bits, zero_offset, ws, na::kScratchBytes, stream);
}
