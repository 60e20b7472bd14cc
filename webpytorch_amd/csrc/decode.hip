// Decode-step operators of a Qwen2-style decoder for gfx950, in fp32 like the reference's
// numpy decode path (`webtorch/llm.py:1258-1304, 1489-1536, 1619-1636`;
// `webtorch/_core.py:1319-1340, 1543-1596, 1764-1787`).
//
// Every position and token id lives in device memory (the decode state), so a whole decode
// step -- embedding, 24 layers, head and argmax -- replays from a captured graph with no host
// work between tokens: the argmax writes the next token id, appends it to the history and
// advances the position.
//
// RoPE uses a cos/sin table [LMAX][HD/2] that the host builds once exactly as the reference
// does (float64 angles, rounded once to fp32), so both sides rotate with identical numbers.
//
// Decode state (int32 words): [0] position of the next token, [1] tokens generated,
// [2] argmax arrival counter (zero between calls), [3] last token id, then per argmax
// workgroup its (value bits, index) partial.
#include <math.h>

#include "miq_common.h"

// The operators that restate the reference's elementwise numpy arithmetic round every product
// and sum separately (no fused multiply-add), so that their results match it bit for bit;
// explicit fmaf() calls (the attention dot products) are unaffected.
#pragma clang fp contract(off)

namespace miq {

constexpr int kArgmaxWGs = 64;

// h[t][:] = embed[ids[t]][:] as fp32
__global__ __launch_bounds__(256) void embed_kernel(const int32_t* __restrict__ ids, const __half* __restrict__ emb,
                                                    float* __restrict__ out, int H, int V) {
  const int t = blockIdx.y;
  const int id = ids[t];
  const int c = blockIdx.x * 256 + threadIdx.x;
  if (c >= H) return;
  out[(size_t)t * H + c] = (id >= 0 && id < V) ? __half2float(emb[(size_t)id * H + c]) : 0.f;
}

// fp32 table: the rows of a dequantized GGUF token_embd, kept exact
__global__ __launch_bounds__(256) void embed_f32_kernel(const int32_t* __restrict__ ids, const float* __restrict__ emb,
                                                        float* __restrict__ out, int H, int V) {
  const int t = blockIdx.y;
  const int id = ids[t];
  const int c = blockIdx.x * 256 + threadIdx.x;
  if (c >= H) return;
  out[(size_t)t * H + c] = (id >= 0 && id < V) ? emb[(size_t)id * H + c] : 0.f;
}

// out = (x / sqrt(mean(x^2) + eps)) * w, one workgroup per row
__global__ __launch_bounds__(256) void rmsnorm_kernel(const float* __restrict__ x, const float* __restrict__ w,
                                                      float* __restrict__ out, int H, float eps) {
  __shared__ float red[4];
  const float* xr = x + (size_t)blockIdx.x * H;
  float* o = out + (size_t)blockIdx.x * H;
  float s = 0.f;
  // rows of up to 8192 values 16-byte aligned: every load of the thread issued before the first
  // is used, the values kept for the scaling pass (a strided loop waits on each load in turn)
  constexpr int U = 8;
  const int n4 = H / 4;
  const bool vec = (H & 3) == 0 && n4 <= U * 256 && (reinterpret_cast<uintptr_t>(xr) & 15) == 0 &&
                   (reinterpret_cast<uintptr_t>(o) & 15) == 0 && (reinterpret_cast<uintptr_t>(w) & 15) == 0;
  float4 v[U];
  if (vec) {
    const float4* x4 = reinterpret_cast<const float4*>(xr);
#pragma unroll
    for (int j = 0; j < U; ++j) {
      const int i = threadIdx.x + j * 256;
      v[j] = i < n4 ? x4[i] : make_float4(0.f, 0.f, 0.f, 0.f);
    }
#pragma unroll
    for (int j = 0; j < U; ++j) {
      s = s + v[j].x * v[j].x;  // products rounded
      s = s + v[j].y * v[j].y;
      s = s + v[j].z * v[j].z;
      s = s + v[j].w * v[j].w;
    }
  } else {
    for (int c = threadIdx.x; c < H; c += 256) s = s + xr[c] * xr[c];
  }
  s = wave_sum(s);
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = s;
  __syncthreads();
  const float ms = ((red[0] + red[1]) + (red[2] + red[3])) / (float)H;
  const float r = sqrtf(ms + eps);
  if (vec) {
    const float4* w4 = reinterpret_cast<const float4*>(w);
    float4* o4 = reinterpret_cast<float4*>(o);
#pragma unroll
    for (int j = 0; j < U; ++j) {
      const int i = threadIdx.x + j * 256;
      if (i < n4) {
        const float4 ww = w4[i];
        o4[i] = make_float4((v[j].x / r) * ww.x, (v[j].y / r) * ww.y, (v[j].z / r) * ww.z, (v[j].w / r) * ww.w);
      }
    }
  } else {
    for (int c = threadIdx.x; c < H; c += 256) o[c] = (xr[c] / r) * w[c];
  }
}

__global__ __launch_bounds__(256) void head_rmsnorm_kernel(float* __restrict__ qkv, const float* __restrict__ qn,
                                                           const float* __restrict__ kn, int T, int NH, int NKV,
                                                           int HD, float eps) {
  const int wid = blockIdx.x * 4 + (threadIdx.x >> 6), lane = threadIdx.x & 63;
  const int nh = NH + NKV;
  if (wid >= T * nh) return;  // whole waves
  const int t = wid / nh, h = wid % nh;
  const float* w = h < NH ? qn : kn;
  if (!w) return;
  float* row = qkv + (size_t)t * (NH + 2 * NKV) * HD + (size_t)h * HD;
  float v[4];
  float s = 0.f;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int d = lane + 64 * i;
    v[i] = d < HD ? row[d] : 0.f;
    s = s + v[i] * v[i];
  }
  s = wave_sum(s);
  const float r = sqrtf(s / (float)HD + eps);
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int d = lane + 64 * i;
    if (d < HD) row[d] = (v[i] / r) * w[d];
  }
}

// Rotate-half RoPE at positions pos0 + t (pos0 read from the device) with the fp32 cos/sin
// table [LMAX][HD/2] (float64 angles rounded once, as the reference builds it), then
// x*cos + rot(x)*sin rounded like the numpy expression. q goes to q_out [T][NH][HD]; k and v
// go into the caches [NKV][LMAX][HD] at their positions (positions past LMAX are not written).
__device__ __forceinline__ float rope1(const float* row, int d, int half, float c, float s) {
  const float rv = d < half ? -row[d + half] : row[d - half];
  return row[d] * c + rv * s;
}

__global__ __launch_bounds__(256) void rope_kv_kernel(const float* __restrict__ qkv, const int32_t* __restrict__ state,
                                                      const float* __restrict__ cos_t, const float* __restrict__ sin_t,
                                                      float* __restrict__ q_out, float* __restrict__ kc,
                                                      float* __restrict__ vc, int NH, int NKV, int HD, int LMAX) {
  const int t = blockIdx.y;
  const int pos = state[0] + t;
  if (pos >= LMAX) return;
  const int W = (NH + 2 * NKV) * HD;
  const float* row = qkv + (size_t)t * W;
  const int half = HD / 2;
  // one value per thread (grid.x covers the row), so no thread waits on a chain of loads
  const int i = blockIdx.x * 256 + threadIdx.x;
  if (i >= W) return;
  const int head = i / HD, d = i - head * HD;
  if (head >= NH + NKV) {  // v: copied into the cache
    vc[((size_t)(head - NH - NKV) * LMAX + pos) * HD + d] = row[i];
    return;
  }
  const int j = d < half ? d : d - half;
  const float y = rope1(row + head * HD, d, half, cos_t[(size_t)pos * half + j], sin_t[(size_t)pos * half + j]);
  if (head < NH) q_out[((size_t)t * NH + head) * HD + d] = y;
  else kc[((size_t)(head - NH) * LMAX + pos) * HD + d] = y;
}

// One decode token: RoPE of its q head and of the kv head's new k, the new k and v written
// into the caches (by the first query head of each kv group), then attention over positions
// 0..pos with the new position's k and v taken from LDS (the other workgroups of the group
// may not have written them yet). A workgroup of 256 threads per query head: a thread per
// position for the scores, then 4 waves over positions x 64 lanes over the head dimension
// for the weighted sum, combined in wave order.
__global__ __launch_bounds__(256) void attention_decode_kernel(
    const float* __restrict__ qkv, const int32_t* __restrict__ state, const float* __restrict__ cos_t,
    const float* __restrict__ sin_t, float* __restrict__ kc, float* __restrict__ vc, float* __restrict__ out, int NH,
    int NKV, int HD, int LMAX, float scale) {
  extern __shared__ float sp[];  // [LMAX] scores -> probabilities
  __shared__ float qs[256], kn[256], vn[256], red[4][256], wred[8];
  const int h = blockIdx.x;
  const int rep = NH / NKV, kv = h / rep;
  const int pos = state[0];
  const int half = HD / 2;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  if (pos >= LMAX) return;  // uniform: the caller never runs past its cache
  const int S = pos + 1;
  for (int d = tid; d < HD; d += 256) {
    const int j = d < half ? d : d - half;
    const float c = cos_t[(size_t)pos * half + j], s = sin_t[(size_t)pos * half + j];
    qs[d] = rope1(qkv + h * HD, d, half, c, s);
    kn[d] = rope1(qkv + (NH + kv) * HD, d, half, c, s);
    vn[d] = qkv[(NH + NKV + kv) * HD + d];
    if (h % rep == 0) {
      kc[((size_t)kv * LMAX + pos) * HD + d] = kn[d];
      vc[((size_t)kv * LMAX + pos) * HD + d] = vn[d];
    }
  }
  __syncthreads();
  const float* K = kc + (size_t)kv * LMAX * HD;
  const float* Vv = vc + (size_t)kv * LMAX * HD;
  float mx = -INFINITY;
  for (int j = tid; j < S; j += 256) {
    const float* kr = j == pos ? kn : K + (size_t)j * HD;
    float a = 0.f;
    for (int d = 0; d < HD; d += 4) {
      const float4 k4 = *reinterpret_cast<const float4*>(kr + d);
      a = fmaf(qs[d], k4.x, a);
      a = fmaf(qs[d + 1], k4.y, a);
      a = fmaf(qs[d + 2], k4.z, a);
      a = fmaf(qs[d + 3], k4.w, a);
    }
    a *= scale;
    sp[j] = a;
    mx = fmaxf(mx, a);
  }
  mx = wave_max(mx);
  if (lane == 0) wred[wave] = mx;
  __syncthreads();
  mx = fmaxf(fmaxf(wred[0], wred[1]), fmaxf(wred[2], wred[3]));
  float sum = 0.f;
  for (int j = tid; j < S; j += 256) {
    const float e = expf(sp[j] - mx);
    sp[j] = e;
    sum += e;
  }
  sum = wave_sum(sum);
  if (lane == 0) wred[4 + wave] = sum;
  __syncthreads();
  sum = (wred[4] + wred[5]) + (wred[6] + wred[7]);
  for (int j = tid; j < S; j += 256) sp[j] = sp[j] / sum;
  __syncthreads();
  for (int d = lane; d < HD; d += 64) {
    float o = 0.f;
    for (int j = wave; j < S; j += 4) o = fmaf(sp[j], j == pos ? vn[d] : Vv[(size_t)j * HD + d], o);
    red[wave][d] = o;
  }
  __syncthreads();
  for (int d = tid; d < HD; d += 256) out[(size_t)h * HD + d] = ((red[0][d] + red[1][d]) + red[2][d]) + red[3][d];
}

// The same for head dimensions 64 and 128 at any cache length, with the cache rows read by
// whole groups of threads of a 1024-thread workgroup: a position's key row is HD / 4 adjacent
// threads (one float4 each, the row's partial dot products summed across the group), so a pass
// covers 4096 / HD positions with coalesced loads, four passes in flight; the weighted sum
// likewise gives each thread a float4 of the head dimension and a residue of the position
// modulo 4096 / HD, four positions in flight, the residues combined in order through LDS.
constexpr int kAttRowThreads = 1024;
template <int HD>
__global__ __launch_bounds__(kAttRowThreads) void attention_decode_rows_kernel(
    const float* __restrict__ qkv, const int32_t* __restrict__ state, const float* __restrict__ cos_t,
    const float* __restrict__ sin_t, float* __restrict__ kc, float* __restrict__ vc, float* __restrict__ out, int NH,
    int NKV, int LMAX, float scale) {
  constexpr int NT = kAttRowThreads, NW = NT / 64, TPP = HD / 4, PPP = NT / TPP, U = 4, HALF = HD / 2;
  extern __shared__ float sp[];  // [LMAX] scores -> probabilities
  __shared__ __align__(16) float qs[HD], kn[HD], vn[HD];
  __shared__ __align__(16) float4 red[PPP][TPP];
  __shared__ float wred[2 * NW];
  const int h = blockIdx.x;
  const int rep = NH / NKV, kv = h / rep;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int c = tid % TPP, r = tid / TPP;
  const float4* K4 = reinterpret_cast<const float4*>(kc + (size_t)kv * LMAX * HD);
  const float4* V4 = reinterpret_cast<const float4*>(vc + (size_t)kv * LMAX * HD);
  const int pos = state[0];
  if (pos >= LMAX) return;  // uniform: the caller never runs past its cache
  const int S = pos + 1;
  if (tid < HD) {
    const int d = tid, j = d < HALF ? d : d - HALF;
    const float c = cos_t[(size_t)pos * HALF + j], s = sin_t[(size_t)pos * HALF + j];
    qs[d] = rope1(qkv + h * HD, d, HALF, c, s);
    kn[d] = rope1(qkv + (NH + kv) * HD, d, HALF, c, s);
    vn[d] = qkv[(NH + NKV + kv) * HD + d];
    if (h % rep == 0) {
      kc[((size_t)kv * LMAX + pos) * HD + d] = kn[d];
      vc[((size_t)kv * LMAX + pos) * HD + d] = vn[d];
    }
  }
  __syncthreads();
  const float4 q4 = reinterpret_cast<const float4*>(qs)[c];
  float mx = -INFINITY;
  for (int j0 = 0; j0 < S; j0 += PPP * U) {
    float4 k4[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int j = min(j0 + u * PPP + r, S - 1);
      k4[u] = j == pos ? reinterpret_cast<const float4*>(kn)[c] : K4[(size_t)j * TPP + c];
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      float a = fmaf(q4.w, k4[u].w, fmaf(q4.z, k4[u].z, fmaf(q4.y, k4[u].y, q4.x * k4[u].x)));
#pragma unroll
      for (int m = TPP / 2; m >= 1; m >>= 1) a += __shfl_xor(a, m, TPP);
      a *= scale;
      const int j = j0 + u * PPP + r;
      if (j < S) {
        if (c == 0) sp[j] = a;
        mx = fmaxf(mx, a);
      }
    }
  }
  mx = wave_max(mx);
  if (lane == 0) wred[wave] = mx;
  __syncthreads();
  mx = wred[0];
#pragma unroll
  for (int w = 1; w < NW; ++w) mx = fmaxf(mx, wred[w]);
  float sum = 0.f;
  for (int j = tid; j < S; j += NT) {
    const float e = expf(sp[j] - mx);
    sp[j] = e;
    sum += e;
  }
  sum = wave_sum(sum);
  if (lane == 0) wred[NW + wave] = sum;
  __syncthreads();
  sum = 0.f;
#pragma unroll
  for (int w = 0; w < NW; ++w) sum += wred[NW + w];
  for (int j = tid; j < S; j += NT) sp[j] = sp[j] / sum;
  __syncthreads();
  float4 o = make_float4(0.f, 0.f, 0.f, 0.f);
  for (int j0 = r; j0 < S; j0 += PPP * U) {
    float4 v4[U];
    float pj[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int j = min(j0 + u * PPP, S - 1);
      v4[u] = j == pos ? reinterpret_cast<const float4*>(vn)[c] : V4[(size_t)j * TPP + c];
      pj[u] = j0 + u * PPP < S ? sp[j] : 0.f;
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      o.x = fmaf(pj[u], v4[u].x, o.x);
      o.y = fmaf(pj[u], v4[u].y, o.y);
      o.z = fmaf(pj[u], v4[u].z, o.z);
      o.w = fmaf(pj[u], v4[u].w, o.w);
    }
  }
  red[r][c] = o;
  __syncthreads();
  if (tid < TPP) {
    float4 t = red[0][tid];
#pragma unroll
    for (int i = 1; i < PPP; ++i) {
      const float4 v = red[i][tid];
      t.x += v.x;
      t.y += v.y;
      t.z += v.z;
      t.w += v.w;
    }
    float* o4 = out + (size_t)h * HD + 4 * tid;
    o4[0] = t.x;
    o4[1] = t.y;
    o4[2] = t.z;
    o4[3] = t.w;
  }
}

// The same for head dimension 64 and caches of at most 256 positions, with every load that does
// not depend on the position issued at entry: the key row of position tid, the value column of
// lane for positions wave + 4 i, and the new q/k/v. The kernel then waits for memory about twice
// (position, then its RoPE row) instead of once per phase. Cache rows past the position are
// read (in bounds) and masked: their scores are -inf and their values never enter the sum. The
// arithmetic and its order are those of attention_decode_kernel.
__global__ __launch_bounds__(256) void attention_decode_small_kernel(
    const float* __restrict__ qkv, const int32_t* __restrict__ state, const float* __restrict__ cos_t,
    const float* __restrict__ sin_t, float* __restrict__ kc, float* __restrict__ vc, float* __restrict__ out, int NH,
    int NKV, int LMAX, float scale) {
  constexpr int HD = 64, HALF = 32;
  __shared__ float qs[HD], kn[HD], vn[HD], red[4][HD], wred[8], sp[256];
  const int h = blockIdx.x;
  const int rep = NH / NKV, kv = h / rep;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const float* K = kc + (size_t)kv * LMAX * HD;
  const float* Vv = vc + (size_t)kv * LMAX * HD;
  float4 kr[HD / 4];
  const float* krow = K + (size_t)min(tid, LMAX - 1) * HD;
#pragma unroll
  for (int i = 0; i < HD / 4; ++i) kr[i] = *reinterpret_cast<const float4*>(krow + 4 * i);
  float vr[64];
#pragma unroll
  for (int i = 0; i < 64; ++i) vr[i] = Vv[(size_t)min(wave + 4 * i, LMAX - 1) * HD + lane];
  const int pos = state[0];
  if (pos >= LMAX) return;  // uniform: the caller never runs past its cache
  const int S = pos + 1;
  if (tid < HD) {
    const int d = tid, j = d < HALF ? d : d - HALF;
    const float c = cos_t[(size_t)pos * HALF + j], s = sin_t[(size_t)pos * HALF + j];
    qs[d] = rope1(qkv + h * HD, d, HALF, c, s);
    kn[d] = rope1(qkv + (NH + kv) * HD, d, HALF, c, s);
    vn[d] = qkv[(NH + NKV + kv) * HD + d];
    if (h % rep == 0) {
      kc[((size_t)kv * LMAX + pos) * HD + d] = kn[d];
      vc[((size_t)kv * LMAX + pos) * HD + d] = vn[d];
    }
  }
  __syncthreads();
  float mx = -INFINITY;
  if (tid < S) {
    float a = 0.f;
#pragma unroll
    for (int i = 0; i < HD / 4; ++i) {
      const float4 k4 = tid == pos ? *reinterpret_cast<const float4*>(kn + 4 * i) : kr[i];
      a = fmaf(qs[4 * i], k4.x, a);
      a = fmaf(qs[4 * i + 1], k4.y, a);
      a = fmaf(qs[4 * i + 2], k4.z, a);
      a = fmaf(qs[4 * i + 3], k4.w, a);
    }
    a *= scale;
    sp[tid] = a;
    mx = a;
  }
  mx = wave_max(mx);
  if (lane == 0) wred[wave] = mx;
  __syncthreads();
  mx = fmaxf(fmaxf(wred[0], wred[1]), fmaxf(wred[2], wred[3]));
  float sum = 0.f;
  if (tid < S) {
    const float e = expf(sp[tid] - mx);
    sp[tid] = e;
    sum = e;
  }
  sum = wave_sum(sum);
  if (lane == 0) wred[4 + wave] = sum;
  __syncthreads();
  sum = (wred[4] + wred[5]) + (wred[6] + wred[7]);
  if (tid < S) sp[tid] = sp[tid] / sum;
  __syncthreads();
  float o = 0.f;
#pragma unroll
  for (int i = 0; i < 64; ++i) {
    const int j = wave + 4 * i;
    if (j < S) o = fmaf(sp[j], j == pos ? vn[lane] : vr[i], o);
  }
  red[wave][lane] = o;
  __syncthreads();
  if (tid < HD) out[(size_t)h * HD + tid] = ((red[0][tid] + red[1][tid]) + red[2][tid]) + red[3][tid];
}

// Causal grouped-query attention: token t (position pos0 + t) of query head h attends to
// cache positions 0 .. pos0 + t of kv head h / (NH / NKV). One wave per (head, token):
// lanes over positions for the scores, lanes over the head dimension for the output.
// scores = (q . k) * scale; p = exp(s - max) / sum; out = sum p v.
__global__ __launch_bounds__(64) void attention_kernel(const float* __restrict__ q, const float* __restrict__ kc,
                                                       const float* __restrict__ vc, const int32_t* __restrict__ state,
                                                       float* __restrict__ out, int NH, int NKV, int HD, int LMAX,
                                                       float scale) {
  extern __shared__ float sp[];  // [LMAX] scores, then probabilities
  __shared__ float qs[256];
  const int h = blockIdx.x, t = blockIdx.y;
  const int lane = threadIdx.x;
  const int kv = h / (NH / NKV);
  int S = state[0] + t + 1;
  S = S > LMAX ? LMAX : S;
  for (int d = lane; d < HD; d += 64) qs[d] = q[((size_t)t * NH + h) * HD + d];
  __syncthreads();
  const float* K = kc + (size_t)kv * LMAX * HD;
  const float* Vv = vc + (size_t)kv * LMAX * HD;
  float mx = -INFINITY;
  for (int j = lane; j < S; j += 64) {
    const float* kr = K + (size_t)j * HD;
    float a = 0.f;
    for (int d = 0; d < HD; d += 4) {
      const float4 k4 = *reinterpret_cast<const float4*>(kr + d);
      a = fmaf(qs[d], k4.x, a);
      a = fmaf(qs[d + 1], k4.y, a);
      a = fmaf(qs[d + 2], k4.z, a);
      a = fmaf(qs[d + 3], k4.w, a);
    }
    a *= scale;
    sp[j] = a;
    mx = fmaxf(mx, a);
  }
  mx = wave_max(mx);
  float sum = 0.f;
  for (int j = lane; j < S; j += 64) {
    const float e = expf(sp[j] - mx);
    sp[j] = e;
    sum += e;
  }
  sum = wave_sum(sum);
  for (int j = lane; j < S; j += 64) sp[j] = sp[j] / sum;
  __syncthreads();
  for (int d = lane; d < HD; d += 64) {
    float o = 0.f;
    for (int j = 0; j < S; ++j) o = fmaf(sp[j], Vv[(size_t)j * HD + d], o);
    out[((size_t)t * NH + h) * HD + d] = o;
  }
}

// out[t][i] = silu(gu[t][i]) * gu[t][I + i], silu(x) = x * (1 / (1 + exp(-x)))
__global__ __launch_bounds__(256) void silu_mul_kernel(const float* __restrict__ gu, float* __restrict__ out, int I) {
  const int t = blockIdx.y;
  const int i = blockIdx.x * 256 + threadIdx.x;
  if (i >= I) return;
  const float g = gu[(size_t)t * 2 * I + i], u = gu[(size_t)t * 2 * I + I + i];
  out[(size_t)t * I + i] = (g * (1.f / (1.f + expf(-g)))) * u;
}

__global__ __launch_bounds__(256) void add_kernel(float* __restrict__ h, const float* __restrict__ y, size_t n) {
  const size_t i = (size_t)blockIdx.x * 256 + threadIdx.x;
  if (i < n) h[i] += y[i];
}

__device__ __forceinline__ bool better(float v, int i, float bv, int bi) {
  return v > bv || (v == bv && i < bi) || (bv != bv && v == v);  // NaN never wins
}

// Greedy pick: argmax (first index on ties) over V logits with kArgmaxWGs workgroups; the
// last to arrive combines the partials in workgroup order, writes the token id (to ids[0], to
// the history at state[1] and to state[3]), advances the position by `advance` and re-arms
// the counter.
__global__ __launch_bounds__(256) void argmax_kernel(const float* __restrict__ logits, int V, int32_t* __restrict__ ids,
                                                     int32_t* __restrict__ history, int hist_len,
                                                     int32_t* __restrict__ state, int advance) {
  __shared__ float bv_s[4];
  __shared__ int bi_s[4];
  __shared__ int is_last;
  const int chunk = (V + gridDim.x - 1) / gridDim.x;
  const int b0 = blockIdx.x * chunk, b1 = min(V, b0 + chunk);
  float bv = -INFINITY;
  int bi = 0x7fffffff;
  for (int i = b0 + threadIdx.x; i < b1; i += 256) {
    const float v = logits[i];
    if (better(v, i, bv, bi)) { bv = v; bi = i; }
  }
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) {
    const float ov = __shfl_xor(bv, o, 64);
    const int oi = __shfl_xor(bi, o, 64);
    if (better(ov, oi, bv, bi)) { bv = ov; bi = oi; }
  }
  if ((threadIdx.x & 63) == 0) { bv_s[threadIdx.x >> 6] = bv; bi_s[threadIdx.x >> 6] = bi; }
  __syncthreads();
  if (threadIdx.x == 0) {
    for (int w = 1; w < 4; ++w)
      if (better(bv_s[w], bi_s[w], bv, bi)) { bv = bv_s[w]; bi = bi_s[w]; }
    int32_t* part = state + 4 + 2 * blockIdx.x;
    __hip_atomic_store(part, __float_as_int(bv), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    __hip_atomic_store(part + 1, bi, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    __builtin_amdgcn_s_waitcnt(0);
    is_last = __hip_atomic_fetch_add(state + 2, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == (int)gridDim.x - 1;
  }
  __syncthreads();
  if (is_last && threadIdx.x < 64) {
    // lane g loads workgroup g's partial (at most 64 workgroups), then a wave arg-max
    float fv = -INFINITY;
    int fi = 0x7fffffff;
    const int g = threadIdx.x;
    if (g < (int)gridDim.x) {
      fv = __int_as_float(__hip_atomic_load(state + 4 + 2 * g, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT));
      fi = __hip_atomic_load(state + 5 + 2 * g, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) {
      const float ov = __shfl_xor(fv, o, 64);
      const int oi = __shfl_xor(fi, o, 64);
      if (better(ov, oi, fv, fi)) { fv = ov; fi = oi; }
    }
    if (threadIdx.x == 0) {
      if (fi >= V) fi = 0;  // all logits NaN
      ids[0] = fi;
      const int step = state[1];
      if (step < hist_len) history[step] = fi;
      state[1] = step + 1;
      state[3] = fi;
      state[0] += advance;
      __hip_atomic_store(state + 2, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
  }
}

}  // namespace miq

using namespace miq;

extern "C" int miq_decode_state_words(void) { return 4 + 2 * kArgmaxWGs; }

extern "C" int miq_embed(const int32_t* ids, const void* embed, float* out, int T, int H, int V, void* stream) {
  MIQ_REQUIRE(T >= 0 && H > 0 && V > 0, MIQ_ERR_INVALID, "embed: T=%d H=%d V=%d", T, H, V);
  if (T == 0) return MIQ_OK;
  MIQ_REQUIRE(ids && embed && out, MIQ_ERR_INVALID, "embed: null pointer");
  hipLaunchKernelGGL(embed_kernel, dim3((H + 255) / 256, T), dim3(256), 0, static_cast<hipStream_t>(stream), ids,
                     static_cast<const __half*>(embed), out, H, V);
  return check_launch("embed");
}

extern "C" int miq_embed_f32(const int32_t* ids, const float* embed, float* out, int T, int H, int V, void* stream) {
  MIQ_REQUIRE(T >= 0 && H > 0 && V > 0, MIQ_ERR_INVALID, "embed_f32: T=%d H=%d V=%d", T, H, V);
  if (T == 0) return MIQ_OK;
  MIQ_REQUIRE(ids && embed && out, MIQ_ERR_INVALID, "embed_f32: null pointer");
  hipLaunchKernelGGL(embed_f32_kernel, dim3((H + 255) / 256, T), dim3(256), 0, static_cast<hipStream_t>(stream), ids,
                     embed, out, H, V);
  return check_launch("embed_f32");
}

extern "C" int miq_rmsnorm(const float* x, const float* w, float* out, int T, int H, float eps, void* stream) {
  MIQ_REQUIRE(T >= 0 && H > 0, MIQ_ERR_INVALID, "rmsnorm: T=%d H=%d", T, H);
  if (T == 0) return MIQ_OK;
  MIQ_REQUIRE(x && w && out, MIQ_ERR_INVALID, "rmsnorm: null pointer");
  hipLaunchKernelGGL(rmsnorm_kernel, dim3(T), dim3(256), 0, static_cast<hipStream_t>(stream), x, w, out, H, eps);
  return check_launch("rmsnorm");
}

extern "C" int miq_head_rmsnorm(float* qkv, const float* qn, const float* kn, int T, int NH, int NKV, int HD, float eps,
                                void* stream) {
  MIQ_REQUIRE(T >= 0 && NH > 0 && NKV > 0 && HD > 0 && HD <= 256, MIQ_ERR_INVALID,
              "head_rmsnorm: T=%d NH=%d NKV=%d HD=%d (HD <= 256)", T, NH, NKV, HD);
  if (T == 0 || (!qn && !kn)) return MIQ_OK;
  MIQ_REQUIRE(qkv, MIQ_ERR_INVALID, "head_rmsnorm: null pointer");
  const int waves = T * (NH + NKV);
  hipLaunchKernelGGL(head_rmsnorm_kernel, dim3((waves + 3) / 4), dim3(256), 0, static_cast<hipStream_t>(stream), qkv,
                     qn, kn, T, NH, NKV, HD, eps);
  return check_launch("head_rmsnorm");
}

extern "C" int miq_rope_kv(const float* qkv, const int32_t* state, const float* cos_tab, const float* sin_tab,
                           float* q_out, float* kcache, float* vcache, int T, int NH, int NKV, int HD, int LMAX,
                           void* stream) {
  MIQ_REQUIRE(T >= 0 && NH > 0 && NKV > 0 && NH % NKV == 0 && HD > 0 && HD % 2 == 0 && LMAX > 0, MIQ_ERR_INVALID,
              "rope_kv: T=%d NH=%d NKV=%d HD=%d LMAX=%d", T, NH, NKV, HD, LMAX);
  if (T == 0) return MIQ_OK;
  MIQ_REQUIRE(qkv && state && cos_tab && sin_tab && q_out && kcache && vcache, MIQ_ERR_INVALID, "rope_kv: null pointer");
  hipLaunchKernelGGL(rope_kv_kernel, dim3(((NH + 2 * NKV) * HD + 255) / 256, T), dim3(256), 0,
                     static_cast<hipStream_t>(stream), qkv, state, cos_tab,
                     sin_tab, q_out, kcache, vcache, NH, NKV, HD, LMAX);
  return check_launch("rope_kv");
}

extern "C" int miq_attention_decode(const float* qkv, const int32_t* state, const float* cos_tab, const float* sin_tab,
                                    float* kcache, float* vcache, float* out, int NH, int NKV, int HD, int LMAX,
                                    float scale, void* stream) {
  MIQ_REQUIRE(NH > 0 && NKV > 0 && NH % NKV == 0 && HD > 0 && HD <= 256 && HD % 4 == 0 && LMAX > 0, MIQ_ERR_INVALID,
              "attention_decode: NH=%d NKV=%d HD=%d LMAX=%d", NH, NKV, HD, LMAX);
  MIQ_REQUIRE((size_t)LMAX * 4 <= 64 * 1024, MIQ_ERR_UNSUPPORTED, "attention_decode: LMAX=%d above 16384", LMAX);
  MIQ_REQUIRE(qkv && state && cos_tab && sin_tab && kcache && vcache && out, MIQ_ERR_INVALID,
              "attention_decode: null pointer");
  MIQ_REQUIRE(aligned(kcache, 16) && aligned(vcache, 16), MIQ_ERR_ALIGN, "attention_decode: caches must be 16-byte aligned");
  if (HD == 64 && LMAX <= 256)
    hipLaunchKernelGGL(attention_decode_small_kernel, dim3(NH), dim3(256), 0, static_cast<hipStream_t>(stream), qkv,
                       state, cos_tab, sin_tab, kcache, vcache, out, NH, NKV, LMAX, scale);
  else if (HD == 64)
    hipLaunchKernelGGL(attention_decode_rows_kernel<64>, dim3(NH), dim3(kAttRowThreads), (size_t)LMAX * 4,
                       static_cast<hipStream_t>(stream), qkv, state, cos_tab, sin_tab, kcache, vcache, out, NH, NKV,
                       LMAX, scale);
  else if (HD == 128)
    hipLaunchKernelGGL(attention_decode_rows_kernel<128>, dim3(NH), dim3(kAttRowThreads), (size_t)LMAX * 4,
                       static_cast<hipStream_t>(stream), qkv, state, cos_tab, sin_tab, kcache, vcache, out, NH, NKV,
                       LMAX, scale);
  else
    hipLaunchKernelGGL(attention_decode_kernel, dim3(NH), dim3(256), (size_t)LMAX * 4, static_cast<hipStream_t>(stream),
                       qkv, state, cos_tab, sin_tab, kcache, vcache, out, NH, NKV, HD, LMAX, scale);
  return check_launch("attention_decode");
}

extern "C" int miq_attention(const float* q, const float* kcache, const float* vcache, const int32_t* state, float* out,
                             int T, int NH, int NKV, int HD, int LMAX, float scale, void* stream) {
  MIQ_REQUIRE(T >= 0 && NH > 0 && NKV > 0 && NH % NKV == 0 && HD > 0 && HD <= 256 && HD % 4 == 0 && LMAX > 0,
              MIQ_ERR_INVALID, "attention: T=%d NH=%d NKV=%d HD=%d LMAX=%d", T, NH, NKV, HD, LMAX);
  if (T == 0) return MIQ_OK;
  MIQ_REQUIRE((size_t)LMAX * 4 <= 64 * 1024, MIQ_ERR_UNSUPPORTED, "attention: LMAX=%d above 16384", LMAX);
  MIQ_REQUIRE(q && kcache && vcache && state && out, MIQ_ERR_INVALID, "attention: null pointer");
  MIQ_REQUIRE(aligned(kcache, 16) && aligned(vcache, 16), MIQ_ERR_ALIGN, "attention: caches must be 16-byte aligned");
  hipLaunchKernelGGL(attention_kernel, dim3(NH, T), dim3(64), (size_t)LMAX * 4, static_cast<hipStream_t>(stream), q,
                     kcache, vcache, state, out, NH, NKV, HD, LMAX, scale);
  return check_launch("attention");
}

extern "C" int miq_silu_mul(const float* gu, float* out, int T, int I, void* stream) {
  MIQ_REQUIRE(T >= 0 && I > 0, MIQ_ERR_INVALID, "silu_mul: T=%d I=%d", T, I);
  if (T == 0) return MIQ_OK;
  MIQ_REQUIRE(gu && out, MIQ_ERR_INVALID, "silu_mul: null pointer");
  hipLaunchKernelGGL(silu_mul_kernel, dim3((I + 255) / 256, T), dim3(256), 0, static_cast<hipStream_t>(stream), gu,
                     out, I);
  return check_launch("silu_mul");
}

extern "C" int miq_add(float* h, const float* y, int64_t n, void* stream) {
  MIQ_REQUIRE(n >= 0, MIQ_ERR_INVALID, "add: n=%lld", (long long)n);
  if (n == 0) return MIQ_OK;
  MIQ_REQUIRE(h && y, MIQ_ERR_INVALID, "add: null pointer");
  hipLaunchKernelGGL(add_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, static_cast<hipStream_t>(stream), h,
                     y, (size_t)n);
  return check_launch("add");
}

extern "C" int miq_argmax_advance(const float* logits, int V, int32_t* ids, int32_t* history, int hist_len,
                                  int32_t* state, int advance, void* stream) {
  MIQ_REQUIRE(V > 0 && hist_len >= 0, MIQ_ERR_INVALID, "argmax: V=%d", V);
  MIQ_REQUIRE(logits && ids && state && (history || hist_len == 0), MIQ_ERR_INVALID, "argmax: null pointer");
  const int wgs = V < 256 * kArgmaxWGs ? (V + 255) / 256 : kArgmaxWGs;
  hipLaunchKernelGGL(argmax_kernel, dim3(wgs), dim3(256), 0, static_cast<hipStream_t>(stream), logits, V, ids, history,
                     hist_len, state, advance);
  return check_launch("argmax");
}
