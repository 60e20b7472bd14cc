// The route buffer of the sparse-MoE kernels: per token its k experts and weights, per expert its
// slots in ascending token order, and the row tiles the grouped GEMMs walk (written by
// miq_moe_route, read by the GPTQ expert GEMMs in moe.hip and the GGUF expert GEMV in
// ggml_gemv.hip).
#pragma once
#include <stddef.h>

namespace miq {

constexpr int kMoeBM = 32;       // rows per tile (two 16-row MFMA blocks)
constexpr int kMoeMaxTK = 4096;  // T * k handled by the single-workgroup router

// Offsets (in 4-byte words) of the route buffer's arrays.
struct RouteLayout {
  size_t topk_e, topk_w, slot_of, sorted_tok, sorted_w, expert_off, ntiles, tiles, slot_max, x_scale, words;
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
  L.slot_max = L.tiles + 4 * (size_t)L.max_tiles;  // [T*k] max |h| of each slot's row (fp32 bits)
  L.x_scale = L.slot_max + tk;                        // [T] row scale of fp32 x
  L.words = L.x_scale + (size_t)T;
  return L;
}

}  // namespace miq
