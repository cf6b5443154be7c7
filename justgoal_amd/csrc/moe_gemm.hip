// Kernel selection for the two expert GEMMs, and the weighted combine.
//
// The GEMMs themselves live in moe_stream.hip (weight streaming, a few pairs per expert),
// moe_tile.hip (LDS-tiled GEMM1) and moe_big.hip (large tiles). Their arithmetic is the same:
// GEMM1 runs one v_mfma_f32_16x16x128_f8f6f4 per 128-wide K scale block and adds its fp32 result
// times hs_scale[kb, token] * s13[e, n/128, kb] to the accumulator
// (goal_full_shape/opus-4.8/moe_fp8_fwd/MOEDIR/main.py:125-132), then applies SwiGLU into bf16 C
// (not requantised to fp8 as the reference solutions do at main.py:151-156); GEMM2 converts the
// W2 e4m3 bytes to bf16 exactly, runs four v_mfma_f32_16x16x32_bf16 per K block (lane group
// g = lane>>4 carries K = 32g + 8c .. +8 for instruction c, the same map on both operands), scales
// by s2[e, h/128, kb] and stores bf16 rows times the pair's routing weight at the pair's
// destination row (out for a token's first local pair, else a partial row for combine_kernel).
//
// The choice of kernel family depends only on shapes (never on routed counts, which stay on the
// device): see launch_gemm1 / launch_gemm2 below.
#include <mutex>

#include "moe_device.h"
#include "moe_kernels.h"

namespace jgmoe {

// Workgroup = (token, 1024 consecutive hidden columns), 8 columns per thread. The token's local
// pair count n comes from its pair_of row (one lane per slot, reduced by a ballot). GEMM2 has
// already stored the first pair's weighted row in out[t] and pairs 2..n in the token's partial
// rows (contiguous, ascending local expert), all bf16; the sum runs in fp32 in that order.
constexpr int kCombineThreads = 128;

__global__ __launch_bounds__(kCombineThreads) void combine_kernel(
    const uint16_t* __restrict__ partial, const int32_t* __restrict__ pair_of, int T, int K,
    int k_local, int H, uint16_t* __restrict__ out) {
  const int H8 = H / 8;
  const int chunks = (H8 + kCombineThreads - 1) / kCombineThreads;
  const int t = blockIdx.x / chunks;
  const int c8 = (blockIdx.x % chunks) * kCombineThreads + threadIdx.x;
  const int lane = threadIdx.x & (kWave - 1);
  const bool local = lane < K && pair_of[(size_t)t * K + lane] >= 0;
  const int n = __popcll(__ballot(local));
  if (n == 1 || c8 >= H8) return;  // one local pair: GEMM2 wrote the final row
  const int c = c8 * 8;
  uint4* dst = (uint4*)(out + (size_t)t * H + c);
  if (n == 0) {
    store_nt16(dst, uint4{0u, 0u, 0u, 0u});
    return;
  }
  float s[8];
  auto add = [&](uint4 v, bool first) {
    const uint32_t u[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const float lo = __uint_as_float(u[i] << 16), hi = __uint_as_float(u[i] & 0xffff0000u);
      s[2 * i] = first ? lo : s[2 * i] + lo;
      s[2 * i + 1] = first ? hi : s[2 * i + 1] + hi;
    }
  };
  // Every row is read once and the output written once: non-temporal loads and stores (T=16384
  // skewed: 216 -> 192 us with the loads, -> 182 us with the stores too).
  add(load_nt16(dst), true);
  const uint16_t* prow = partial + (size_t)t * (k_local - 1) * H + c;
  for (int j = 0; j + 1 < n; ++j) add(load_nt16(prow + (size_t)j * H), false);
  uint4 o;
  o.x = (uint32_t)float_to_bf16_bits(s[0]) | ((uint32_t)float_to_bf16_bits(s[1]) << 16);
  o.y = (uint32_t)float_to_bf16_bits(s[2]) | ((uint32_t)float_to_bf16_bits(s[3]) << 16);
  o.z = (uint32_t)float_to_bf16_bits(s[4]) | ((uint32_t)float_to_bf16_bits(s[5]) << 16);
  o.w = (uint32_t)float_to_bf16_bits(s[6]) | ((uint32_t)float_to_bf16_bits(s[7]) << 16);
  store_nt16(dst, o);
}

// Kernel families by rows_hint = T*top_k/E (expected pairs per expert), per GEMM, from sweeps
// over DS-V3 T = 16..16384 and Qwen3-style T = 32..1024. GEMM1 streams weights up to 4 expected
// rows, uses the LDS-tiled kernels up to 15 and the large-tile kernel from 16 (64-row tiles up to
// 63, 128-row tiles from 64; moe_big.hip has the measurements). GEMM2 uses the LDS-tiled
// kernel up to 7 expected rows (16-row tiles at <= 1, 32-row tiles above) and the large-tile
// kernel from 8 (64-row tiles up to 63, 128-row tiles from 64); the streaming GEMM2 remains the
// fallback for shapes the tiled kernel does not take.
// The streaming kernels' 16-row items re-stream an expert's weights once per 16 rows, so they
// only win while segments are that short; the tiled GEMM2 shares one staged C tile among four
// waves and streams each weight block once per 32 rows. Against streaming up to 4 rows and large
// tiles above, it took DS-V3 T=16 from 64.6 to 61.7 us, T=64 from 131.8 to 126.1, T=128 from
// 170.4 to 158.6, T=256 from 190.1 to 173.9 and Qwen3 T=128 from 467 to 434 (T=512, 16 rows:
// level with the large tiles; 64-row tiled items from 17 rows lost to them, 299 vs 252 at 24).
// The 64-row large tiles (moe_big.hip) then moved the switch from 16 to 7 expected rows: DS-V3
// T=256 (8 rows) 172.2 -> 170.4 us, T=384 186.1 -> 178.9, T=512 226.4 -> 210.0; Qwen3-style
// T=128 432.3 -> 428.6, T=256 461.7 -> 452.2; at 6 rows the tiled kernel stays ahead (DS-V3 T=192
// 163.5 against 168.3).
// Since the streaming GEMM1 deals its items wave-index major (every CU busy when a batch has
// fewer items than the grid has waves), it beats the LDS-tiled GEMM1 up to 4 expected rows
// (whole call, DS-V3: T=64 126.7 -> 125.6 us, T=96 157.9 -> 151.4, T=128 158.3 -> 152.6;
// Qwen3-style T=32 367.2 -> 358.1, T=64 416.5 -> 405.3); level at 5 (DS-V3 T=160, Qwen3 T=80)
// and behind from 6 (DS-V3 T=176 162.9 against 166.8, T=192 164.2 against 172.6, Qwen3 T=96
// 425.5 against 428.2, T=128 427.4 against 438.5).
constexpr int kStreamMaxRows = 4;
constexpr int kBigRows = 16;
constexpr int kG2TileMaxRows = 7;

// M sub-tiles (of 16 rows) per work item for an expected segment length.
static inline int stream_mt(int rows_hint) { return rows_hint <= 16 ? 1 : rows_hint <= 32 ? 2 : 4; }

hipError_t launch_gemm1(const uint8_t* hs, const float* hs_scale, const uint8_t* w13,
                        const float* s13, const int32_t* counts, const int32_t* offsets,
                        const int32_t* sorted_tok, uint16_t* C, int T, int H, int I, int E_l,
                        int max_pairs, int rows_hint, hipStream_t stream) {
  if (max_pairs <= 0) return hipSuccess;
  if (rows_hint <= kStreamMaxRows)
    return launch_gemm1_stream(hs, hs_scale, w13, s13, counts, offsets, sorted_tok, C, T, H, I,
                               E_l, max_pairs, stream_mt(rows_hint), stream);
  if (rows_hint >= kBigRows) {
    const hipError_t b = launch_gemm1_big(hs, hs_scale, w13, s13, counts, offsets, sorted_tok, C,
                                          T, H, I, E_l, max_pairs, rows_hint, stream);
    if (b != hipErrorNotSupported) return b;
  }
  const hipError_t e = launch_gemm1_tile(hs, hs_scale, w13, s13, counts, offsets, sorted_tok, C,
                                         T, H, I, E_l, max_pairs, stream);
  if (e != hipErrorNotSupported) return e;
  return launch_gemm1_stream(hs, hs_scale, w13, s13, counts, offsets, sorted_tok, C, T, H, I, E_l,
                             max_pairs, 4, stream);
}

hipError_t launch_gemm2(const uint16_t* C, const uint8_t* w2, const float* s2,
                        const int32_t* counts, const int32_t* offsets, const float* sorted_w,
                        Gemm2Out dst, int H, int I, int E_l, int max_pairs, int rows_hint,
                        hipStream_t stream) {
  if (max_pairs <= 0) return hipSuccess;
  if (rows_hint <= kG2TileMaxRows) {
    const hipError_t t = launch_gemm2_tile(C, w2, s2, counts, offsets, sorted_w, dst, H, I, E_l,
                                           max_pairs, rows_hint <= 1 ? 1 : 2, stream);
    if (t != hipErrorNotSupported) return t;
  }
  if (rows_hint > kG2TileMaxRows) {
    const hipError_t b = launch_gemm2_big(C, w2, s2, counts, offsets, sorted_w, dst, H, I, E_l,
                                          max_pairs, rows_hint, stream);
    if (b != hipErrorNotSupported) return b;
  }
  return launch_gemm2_stream(C, w2, s2, counts, offsets, sorted_w, dst, H, I, E_l, max_pairs,
                             4, stream);
}

int device_cu_count() {
  constexpr int kMaxDevices = 64;
  static std::once_flag flags[kMaxDevices];
  static int cus[kMaxDevices];
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) return 256;
  std::call_once(flags[dev], [dev] {
    int n = 0;
    cus[dev] = hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) == hipSuccess &&
                       n > 0
                   ? n
                   : 256;
  });
  return cus[dev];
}

hipError_t launch_combine(const uint16_t* partial, const int32_t* pair_of, int T, int K,
                          int k_local, int H, uint16_t* out, hipStream_t stream) {
  if (T == 0) return hipSuccess;
  const long long chunks = (H / 8 + kCombineThreads - 1) / kCombineThreads;
  combine_kernel<<<dim3((unsigned)(T * chunks)), kCombineThreads, 0, stream>>>(
      partial, pair_of, T, K, k_local, H, out);
  return hipGetLastError();
}

}  // namespace jgmoe
