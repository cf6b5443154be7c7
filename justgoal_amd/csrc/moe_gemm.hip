// Grouped expert GEMMs and the weighted combine.
//
// GEMM1 (W13) + SwiGLU. For one M-tile of an expert's segment (BM = 16*MT pairs) and 64*NW
// columns of C, each wave owns NW column tiles of 16 in both halves of W13 (X1 rows c, X2 rows
// I + c), so the SwiGLU epilogue pairs accumulators that sit in the same lane and register.
// K runs over H in 128-wide scale blocks; one v_mfma_f32_16x16x128_f8f6f4 covers a block exactly,
// its fp32 result is scaled by hs_scale[kb, token] * s13[e, n/128, kb] and added to the running
// accumulator (reference: goal_full_shape/opus-4.8/moe_fp8_fwd/MOEDIR/main.py:125-132).
// C is kept in bf16 (not requantised to fp8 as the reference solutions do at main.py:151-156).
//
// GEMM2 (W2). Same tiling over (pairs x H); C rows are bf16, W2 e4m3 bytes are converted to bf16
// in registers (exact) and fed to v_mfma_f32_16x16x32_bf16; each 128-wide K block is scaled by
// s2[e, h/128, kb]. The epilogue multiplies by the pair's routing weight and stores fp32 rows.
//
// Operands stream straight from HBM into registers (weights are read once per M-tile, so the
// LDS would only add a hop); a register double buffer keeps one K block of loads in flight.
//
// K mapping: within a 128-wide K block, lane group g = lane>>4 holds the 32 contiguous K values
// [32g, 32g+32) of its row for both operands. For the bf16 MFMA (K=32 per instruction) chunk c
// of those 32 values is fed to instruction c, so instruction c covers K = {32g + 8c .. +8 : g}.
// Because A and B use the same map, each output still sums over every K exactly once.
#include "moe_device.h"
#include "moe_kernels.h"

namespace jgmoe {

template <int MT, int NW>
struct G1Stage {
  v8i a[MT];
  v8i b1[NW], b2[NW];
  float sa[MT][4];
  float sw1, sw2;
};

template <int MT, int NW>
__global__ __launch_bounds__(256) void gemm1_swiglu_kernel(
    const uint8_t* __restrict__ hs, const float* __restrict__ hs_scale,
    const uint8_t* __restrict__ w13, const float* __restrict__ s13,
    const int32_t* __restrict__ counts, const int32_t* __restrict__ offsets,
    const int32_t* __restrict__ sorted_tok, uint16_t* __restrict__ C, int T, int H, int I,
    int E_l) {
  constexpr int BM = 16 * MT;
  int e, m0;
  if (!find_m_tile(counts, E_l, BM, blockIdx.x, e, m0)) return;
  const int lane = threadIdx.x & (kWave - 1), wave = threadIdx.x / kWave;
  const int r16 = lane & 15, g = lane >> 4;
  const int cnt = counts[e], seg = offsets[e];
  const int c0 = blockIdx.y * (64 * NW) + wave * (16 * NW);
  const int NKB = H / kBlock;

  const uint8_t* arow[MT];
  bool aval[MT];
  int etok[MT][4];
  bool evalid[MT][4];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) {
    const int r = m0 + mt * 16 + r16;
    aval[mt] = r < cnt;
    const int tok = aval[mt] ? sorted_tok[seg + r] : 0;
    arow[mt] = hs + (size_t)tok * H + 32 * g;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int re = m0 + mt * 16 + 4 * g + i;
      evalid[mt][i] = re < cnt;
      etok[mt][i] = evalid[mt][i] ? sorted_tok[seg + re] : 0;
    }
  }
  const uint8_t* wrow1 = w13 + ((size_t)e * 2 * I + c0 + r16) * H + 32 * g;
  const size_t half = (size_t)I * H;
  const float* sc1 = s13 + ((size_t)e * (2 * I / kBlock) + c0 / kBlock) * NKB;
  const float* sc2 = s13 + ((size_t)e * (2 * I / kBlock) + (I + c0) / kBlock) * NKB;

  v4f acc1[MT][NW], acc2[MT][NW];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt)
#pragma unroll
    for (int j = 0; j < NW; ++j) {
      acc1[mt][j] = v4f{0.f, 0.f, 0.f, 0.f};
      acc2[mt][j] = v4f{0.f, 0.f, 0.f, 0.f};
    }

  auto load = [&](int kb, G1Stage<MT, NW>& st) {
    const v8i zero = {0, 0, 0, 0, 0, 0, 0, 0};
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
      st.a[mt] = aval[mt] ? *(const v8i*)(arow[mt] + kb * kBlock) : zero;
#pragma unroll
    for (int j = 0; j < NW; ++j) {
      const uint8_t* p = wrow1 + (size_t)j * 16 * H + kb * kBlock;
      st.b1[j] = *(const v8i*)p;
      st.b2[j] = *(const v8i*)(p + half);
    }
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
      for (int i = 0; i < 4; ++i)
        st.sa[mt][i] = evalid[mt][i] ? hs_scale[(size_t)kb * T + etok[mt][i]] : 0.f;
    st.sw1 = sc1[kb];
    st.sw2 = sc2[kb];
  };
  auto compute = [&](const G1Stage<MT, NW>& st) {
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
      float f1[4], f2[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        f1[i] = st.sa[mt][i] * st.sw1;
        f2[i] = st.sa[mt][i] * st.sw2;
      }
#pragma unroll
      for (int j = 0; j < NW; ++j) {
        const v4f p = mfma_f8_16x16x128(st.a[mt], st.b1[j]);
        const v4f q = mfma_f8_16x16x128(st.a[mt], st.b2[j]);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          acc1[mt][j][i] = fmaf(p[i], f1[i], acc1[mt][j][i]);
          acc2[mt][j][i] = fmaf(q[i], f2[i], acc2[mt][j][i]);
        }
      }
    }
  };

  G1Stage<MT, NW> s0, s1;
  load(0, s0);
  for (int kb = 0; kb < NKB; kb += 2) {
    if (kb + 1 < NKB) load(kb + 1, s1);
    compute(s0);
    if (kb + 2 < NKB) load(kb + 2, s0);
    if (kb + 1 < NKB) compute(s1);
  }

#pragma unroll
  for (int mt = 0; mt < MT; ++mt)
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int r = m0 + mt * 16 + 4 * g + i;
      if (r >= cnt) continue;
      uint16_t* crow = C + (size_t)(seg + r) * I + c0 + r16;
#pragma unroll
      for (int j = 0; j < NW; ++j) {
        const float x1 = acc1[mt][j][i], x2 = acc2[mt][j][i];
        crow[16 * j] = float_to_bf16_bits(x1 * (x2 / (1.0f + __expf(-x2))));
      }
    }
}

template <int MT, int NW>
struct G2Stage {
  uint4 a[MT][4];
  v8i b[NW];
  float sw;
};

__device__ __forceinline__ v8bf as_v8bf(const uint4& u) { return __builtin_bit_cast(v8bf, u); }

template <int MT, int NW>
__global__ __launch_bounds__(256) void gemm2_kernel(
    const uint16_t* __restrict__ C, const uint8_t* __restrict__ w2, const float* __restrict__ s2,
    const int32_t* __restrict__ counts, const int32_t* __restrict__ offsets,
    const float* __restrict__ sorted_w, float* __restrict__ partial, int H, int I, int E_l) {
  constexpr int BM = 16 * MT;
  int e, m0;
  if (!find_m_tile(counts, E_l, BM, blockIdx.x, e, m0)) return;
  const int lane = threadIdx.x & (kWave - 1), wave = threadIdx.x / kWave;
  const int r16 = lane & 15, g = lane >> 4;
  const int cnt = counts[e], seg = offsets[e];
  const int h0 = blockIdx.y * (64 * NW) + wave * (16 * NW);
  const int NKB = I / kBlock;

  const uint16_t* crow[MT];
  bool aval[MT];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) {
    const int r = m0 + mt * 16 + r16;
    aval[mt] = r < cnt;
    crow[mt] = C + (size_t)(seg + (aval[mt] ? r : 0)) * I + 32 * g;
  }
  const uint8_t* wrow = w2 + ((size_t)e * H + h0 + r16) * I + 32 * g;
  const float* sc = s2 + ((size_t)e * (H / kBlock) + h0 / kBlock) * NKB;

  v4f acc[MT][NW];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt)
#pragma unroll
    for (int j = 0; j < NW; ++j) acc[mt][j] = v4f{0.f, 0.f, 0.f, 0.f};

  auto load = [&](int kb, G2Stage<MT, NW>& st) {
    const uint4 zero = {0u, 0u, 0u, 0u};
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
      for (int c = 0; c < 4; ++c)
        st.a[mt][c] = aval[mt] ? *(const uint4*)(crow[mt] + kb * kBlock + 8 * c) : zero;
#pragma unroll
    for (int j = 0; j < NW; ++j) st.b[j] = *(const v8i*)(wrow + (size_t)j * 16 * I + kb * kBlock);
    st.sw = sc[kb];
  };
  auto compute = [&](const G2Stage<MT, NW>& st) {
#pragma unroll
    for (int j = 0; j < NW; ++j) {
      v8bf bc[4];
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        v2bf p0, p1, p2, p3;
        fp8x4_to_bf16x4(st.b[j][2 * c], p0, p1);
        fp8x4_to_bf16x4(st.b[j][2 * c + 1], p2, p3);
        bc[c] = v8bf{p0[0], p0[1], p1[0], p1[1], p2[0], p2[1], p3[0], p3[1]};
      }
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) {
        v4f t = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int c = 0; c < 4; ++c) t = mfma_bf16_16x16x32(as_v8bf(st.a[mt][c]), bc[c], t);
#pragma unroll
        for (int i = 0; i < 4; ++i) acc[mt][j][i] = fmaf(t[i], st.sw, acc[mt][j][i]);
      }
    }
  };

  G2Stage<MT, NW> s0, s1;
  load(0, s0);
  for (int kb = 0; kb < NKB; kb += 2) {
    if (kb + 1 < NKB) load(kb + 1, s1);
    compute(s0);
    if (kb + 2 < NKB) load(kb + 2, s0);
    if (kb + 1 < NKB) compute(s1);
  }

#pragma unroll
  for (int mt = 0; mt < MT; ++mt)
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int r = m0 + mt * 16 + 4 * g + i;
      if (r >= cnt) continue;
      const int p = seg + r;
      const float wp = sorted_w[p];
      float* orow = partial + (size_t)p * H + h0 + r16;
#pragma unroll
      for (int j = 0; j < NW; ++j) orow[16 * j] = acc[mt][j][i] * wp;
    }
}

// One thread per (token, 8 consecutive hidden columns).
__global__ __launch_bounds__(256) void combine_kernel(const float* __restrict__ partial,
                                                      const int32_t* __restrict__ pair_of, int T,
                                                      int K, int H, uint16_t* __restrict__ out) {
  const int H8 = H / 8;
  const long long gid = (long long)blockIdx.x * 256 + threadIdx.x;
  if (gid >= (long long)T * H8) return;
  const int t = (int)(gid / H8);
  const int c = (int)(gid % H8) * 8;
  int p[kMaxTopK];
  int n = 0;
  for (int k = 0; k < K; ++k) {
    const int q = pair_of[(size_t)t * K + k];
    if (q >= 0) {
      // insertion into the ascending list (pair rows ascend with the local expert)
      int j = n++;
      while (j > 0 && p[j - 1] > q) {
        p[j] = p[j - 1];
        --j;
      }
      p[j] = q;
    }
  }
  float s[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
  for (int j = 0; j < n; ++j) {
    const float4* src = (const float4*)(partial + (size_t)p[j] * H + c);
    const float4 u = src[0], v = src[1];
    s[0] += u.x; s[1] += u.y; s[2] += u.z; s[3] += u.w;
    s[4] += v.x; s[5] += v.y; s[6] += v.z; s[7] += v.w;
  }
  uint4 o;
  o.x = (uint32_t)float_to_bf16_bits(s[0]) | ((uint32_t)float_to_bf16_bits(s[1]) << 16);
  o.y = (uint32_t)float_to_bf16_bits(s[2]) | ((uint32_t)float_to_bf16_bits(s[3]) << 16);
  o.z = (uint32_t)float_to_bf16_bits(s[4]) | ((uint32_t)float_to_bf16_bits(s[5]) << 16);
  o.w = (uint32_t)float_to_bf16_bits(s[6]) | ((uint32_t)float_to_bf16_bits(s[7]) << 16);
  *(uint4*)(out + (size_t)t * H + c) = o;
}

#ifndef JG_STREAM_MAX_ROWS
#define JG_STREAM_MAX_ROWS 16
#endif

// M sub-tiles (of 16 rows) per streaming item for an expected segment length.
static inline int stream_mt(int rows_hint) { return rows_hint <= 16 ? 1 : rows_hint <= 32 ? 2 : 4; }

static inline int m_slots(int max_pairs, int bm, int E_l) {
  return (max_pairs + bm - 1) / bm + (E_l < max_pairs ? E_l : max_pairs);
}

hipError_t launch_gemm1(const uint8_t* hs, const float* hs_scale, const uint8_t* w13,
                        const float* s13, const int32_t* counts, const int32_t* offsets,
                        const int32_t* sorted_tok, uint16_t* C, int T, int H, int I, int E_l,
                        int max_pairs, int rows_hint, hipStream_t stream) {
  if (max_pairs <= 0) return hipSuccess;
  if (rows_hint <= JG_STREAM_MAX_ROWS) {
    return launch_gemm1_stream(hs, hs_scale, w13, s13, counts, offsets, sorted_tok, C, T, H, I,
                               E_l, max_pairs, stream_mt(rows_hint), stream);
  } else {
    constexpr int MT = 4, NW = 2;
    const dim3 grid(m_slots(max_pairs, 16 * MT, E_l), I / (64 * NW));
    gemm1_swiglu_kernel<MT, NW><<<grid, 256, 0, stream>>>(hs, hs_scale, w13, s13, counts,
                                                          offsets, sorted_tok, C, T, H, I, E_l);
  }
  return hipGetLastError();
}

hipError_t launch_gemm2(const uint16_t* C, const uint8_t* w2, const float* s2,
                        const int32_t* counts, const int32_t* offsets, const float* sorted_w,
                        float* partial, int H, int I, int E_l, int max_pairs, int rows_hint, hipStream_t stream) {
  if (max_pairs <= 0) return hipSuccess;
  if (rows_hint <= JG_STREAM_MAX_ROWS) {
    return launch_gemm2_stream(C, w2, s2, counts, offsets, sorted_w, partial, H, I, E_l,
                               max_pairs, stream_mt(rows_hint), stream);
  } else {
    constexpr int MT = 4, NW = 2;
    const dim3 grid(m_slots(max_pairs, 16 * MT, E_l), H / (64 * NW));
    gemm2_kernel<MT, NW><<<grid, 256, 0, stream>>>(C, w2, s2, counts, offsets, sorted_w, partial,
                                                   H, I, E_l);
  }
  return hipGetLastError();
}

hipError_t launch_combine(const float* partial, const int32_t* pair_of, int T, int K, int H,
                          uint16_t* out, hipStream_t stream) {
  const long long n = (long long)T * (H / 8);
  if (n == 0) return hipSuccess;
  combine_kernel<<<dim3((unsigned)((n + 255) / 256)), 256, 0, stream>>>(partial, pair_of, T, K, H,
                                                                        out);
  return hipGetLastError();
}

}  // namespace jgmoe
