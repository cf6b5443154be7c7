// Host-side launchers of the MoE kernels (internal to the library; the public ABI is
// include/justgoal_moe.h).
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace jgmoe {

constexpr int ROUTING_DS = 0;
constexpr int ROUTING_SOFTMAX = 1;

// Routing. Writes topk_idx / topk_w and the count rows `hist` [route_chunks(T), E_l].
hipError_t launch_route(const float* logits, const uint16_t* bias, int T, int E, int n_group,
                        int topk_group, int top_k, int method, float rsf, int local_offset,
                        int E_l, int32_t* topk_idx, float* topk_w, int32_t* hist,
                        hipStream_t stream);

// Segment layout (counts, offsets, sorted tokens/weights, pair map) from the count rows, and
// each pair's GEMM2 destination row (pair_dst, encoded as described at launch_gemm2).
hipError_t launch_permute(const int32_t* topk_idx, const float* topk_w, const int32_t* hist,
                          int T, int K, int local_offset, int E_l, int32_t* counts,
                          int32_t* offsets, int32_t* sorted_tok, float* sorted_w,
                          int32_t* pair_dst, int32_t* pair_of, hipStream_t stream);

// Number of routing workgroups (4 tokens each up to T = 2048, 16 above) = rows of the chunk count
// table.
int route_chunks(int T);

// Grouped GEMM1 (W13) with the SwiGLU epilogue: C[p, :] = bf16(X1 * silu(X2)) for every pair p.
// max_pairs bounds the number of pairs (sizes the grid; surplus workgroups exit at once);
// rows_hint, the expected pairs per expert under uniform routing, picks the tile shape.
hipError_t launch_gemm1(const uint8_t* hs, const float* hs_scale, const uint8_t* w13,
                        const float* s13, const int32_t* counts, const int32_t* offsets,
                        const int32_t* sorted_tok, uint16_t* C, int T, int H, int I, int E_l,
                        int max_pairs, int rows_hint, hipStream_t stream);

// Grouped GEMM2 (W2): row = bf16(w_p * (C[p, :] @ W2[e]^T)), stored at the pair's destination
// d = pair_dst[p]: out row d when d >= 0 (the token's first local pair in ascending expert
// order), else partial row -1 - d (its later pairs; bf16 [T * (min(top_k, E_l) - 1), H]).
struct Gemm2Out {
  const int32_t* pair_dst;
  uint16_t* out;
  uint16_t* partial;
};
hipError_t launch_gemm2(const uint16_t* C, const uint8_t* w2, const float* s2,
                        const int32_t* counts, const int32_t* offsets, const float* sorted_w,
                        Gemm2Out dst, int H, int I, int E_l, int max_pairs, int rows_hint,
                        hipStream_t stream);

// Persistent weight-streaming variants for segments of at most a few 16-row tiles.
hipError_t launch_gemm1_stream(const uint8_t* hs, const float* hs_scale, const uint8_t* w13,
                               const float* s13, const int32_t* counts, const int32_t* offsets,
                               const int32_t* sorted_tok, uint16_t* C, int T, int H, int I,
                               int E_l, int max_pairs, int mt, hipStream_t stream);
hipError_t launch_gemm2_stream(const uint16_t* C, const uint8_t* w2, const float* s2,
                               const int32_t* counts, const int32_t* offsets,
                               const float* sorted_w, Gemm2Out dst, int H, int I, int E_l,
                               int max_pairs, int mt, hipStream_t stream);

// Large-tile variants (BM x BN per workgroup, both operands shared through LDS) for long
// segments. Return hipErrorNotSupported for shapes they do not tile.
hipError_t launch_gemm1_big(const uint8_t* hs, const float* hs_scale, const uint8_t* w13,
                            const float* s13, const int32_t* counts, const int32_t* offsets,
                            const int32_t* sorted_tok, uint16_t* C, int T, int H, int I, int E_l,
                            int max_pairs, int rows_hint, hipStream_t stream);
hipError_t launch_gemm2_big(const uint16_t* C, const uint8_t* w2, const float* s2,
                            const int32_t* counts, const int32_t* offsets, const float* sorted_w,
                            Gemm2Out dst, int H, int I, int E_l, int max_pairs, int rows_hint,
                            hipStream_t stream);

// LDS-tiled variants for longer segments (mt = 16-row sub-tiles per workgroup tile).
hipError_t launch_gemm1_tile(const uint8_t* hs, const float* hs_scale, const uint8_t* w13,
                             const float* s13, const int32_t* counts, const int32_t* offsets,
                             const int32_t* sorted_tok, uint16_t* C, int T, int H, int I, int E_l,
                             int max_pairs, hipStream_t stream);
// LDS-tiled GEMM2 (mt = 16-row sub-tiles per workgroup tile).
hipError_t launch_gemm2_tile(const uint16_t* C, const uint8_t* w2, const float* s2,
                             const int32_t* counts, const int32_t* offsets, const float* sorted_w,
                             Gemm2Out dst, int H, int I, int E_l, int max_pairs, int mt,
                             hipStream_t stream);

// Compute units of the current device, queried once per device (thread-safe); 256 when the
// query fails. Sizes the persistent grids.
int device_cu_count();

// Finishes the output after GEMM2: a token with no local pair gets a zero row; one with n >= 2
// gets bf16(out[t] + partial rows 0..n-2 of t, summed in fp32 in that order, i.e. ascending
// local expert); a token with exactly one local pair keeps the row GEMM2 wrote.
hipError_t launch_combine(const uint16_t* partial, const int32_t* pair_of, int T, int K,
                          int k_local, int H, uint16_t* out, hipStream_t stream);

// Activation quantisation: bf16 [T, H] -> e4m3 [T, H] and fp32 scales [H/128, T] (1x128 blocks,
// scale = amax / 448). H must be a multiple of 128.
hipError_t launch_quantize_activations(const uint16_t* x, int T, int H, uint8_t* q, float* scale,
                                       hipStream_t stream);

}  // namespace jgmoe
