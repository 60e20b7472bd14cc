// Asymmetric min-max group quantizer (GPTQ layout, zero_offset 0), bit-exact with the
// reference's float32 numpy arithmetic: scale = (max - min) / qmax (0 -> 1e-8),
// zero = clip(rint(-min / scale), 0, qmax), code = clip(rint(w / scale) + zero, 0, qmax).
// Division is IEEE round-to-nearest and rint is round-half-even, as numpy's float32 ops.
#include "miq_common.h"

namespace miq {

// One thread per (group, column). W is [K][N] (from_out_in = 0) or [N][K] (= 1), fp16/fp32.
// Codes are packed per thread (a column's rows are in one thread); zero points are packed
// along N through LDS by the lane that owns the first column of each word.
template <int BITS, typename WT>
__global__ __launch_bounds__(256) void gptq_quantize_kernel(const WT* __restrict__ W, int from_out_in, int K, int N,
                                                            int gs, uint32_t* __restrict__ qweight,
                                                            uint32_t* __restrict__ qzeros, float* __restrict__ scales) {
  constexpr int PER = 32 / BITS;
  constexpr int QMAX = (1 << BITS) - 1;
  __shared__ uint32_t zs[256];
  const int n = blockIdx.x * blockDim.x + threadIdx.x;
  const int g = blockIdx.y;
  uint32_t zp = 0;
  if (n < N) {
    auto at = [&](int k) -> float {
      return to_f32(from_out_in ? W[(size_t)n * K + k] : W[(size_t)k * N + n]);
    };
    const int k0 = g * gs;
    float lo = at(k0), hi = lo;
    for (int k = k0 + 1; k < k0 + gs; ++k) {
      const float v = at(k);
      lo = fminf(lo, v);
      hi = fmaxf(hi, v);
    }
    float s = (hi - lo) / (float)QMAX;
    if (s == 0.f) s = 1e-8f;
    float zf = rintf(-lo / s);
    zf = fminf(fmaxf(zf, 0.f), (float)QMAX);
    zp = (uint32_t)zf;
    scales[(size_t)g * N + n] = s;
    for (int r = k0 / PER; r < (k0 + gs) / PER; ++r) {
      uint32_t word = 0;
#pragma unroll
      for (int j = 0; j < PER; ++j) {
        float c = rintf(at(r * PER + j) / s) + zf;
        c = fminf(fmaxf(c, 0.f), (float)QMAX);
        word |= (uint32_t)c << (j * BITS);
      }
      qweight[(size_t)r * N + n] = word;
    }
  }
  zs[threadIdx.x] = zp;
  __syncthreads();
  if (n < N && (n % PER) == 0) {
    uint32_t word = 0;
#pragma unroll
    for (int j = 0; j < PER; ++j) word |= zs[threadIdx.x + j] << (j * BITS);
    qzeros[(size_t)g * (N / PER) + n / PER] = word;
  }
}

}  // namespace miq

using namespace miq;

extern "C" int miq_gptq_quantize(const void* W, int w_dtype, int from_out_in, int K, int N, int gs, int bits,
                                 int32_t* qweight, int32_t* qzeros, float* scales, void* stream) {
  MIQ_REQUIRE(bits == 4 || bits == 8, MIQ_ERR_UNSUPPORTED, "gptq_quantize: bits=%d", bits);
  const int per = 32 / bits;
  MIQ_REQUIRE(K > 0 && N > 0 && gs > 0 && K % gs == 0 && K % per == 0 && N % per == 0 && gs % per == 0,
              MIQ_ERR_INVALID, "gptq_quantize: dims must divide group/pack size (K=%d N=%d gs=%d)", K, N, gs);
  MIQ_REQUIRE(W && qweight && qzeros && scales, MIQ_ERR_INVALID, "gptq_quantize: null pointer");
  dim3 grid((N + 255) / 256, K / gs);
  hipStream_t st = static_cast<hipStream_t>(stream);
  uint32_t* qw = reinterpret_cast<uint32_t*>(qweight);
  uint32_t* qz = reinterpret_cast<uint32_t*>(qzeros);
#define MIQ_Q(B, T) hipLaunchKernelGGL((gptq_quantize_kernel<B, T>), grid, dim3(256), 0, st, \
                                       static_cast<const T*>(W), from_out_in, K, N, gs, qw, qz, scales)
  if (bits == 4) {
    if (w_dtype == MIQ_F16) MIQ_Q(4, __half); else MIQ_Q(4, float);
  } else {
    if (w_dtype == MIQ_F16) MIQ_Q(8, __half); else MIQ_Q(8, float);
  }
#undef MIQ_Q
  return check_launch("gptq_quantize");
}
