// Weight-streaming grouped GEMMs for small per-expert segments (decode-sized batches).
//
// When an expert holds a handful of pairs, every weight byte is used by at most one 16-row MFMA
// tile, so the GEMMs are HBM streams: the kernels must keep enough bytes in flight per CU and
// must not leave CUs idle. Both kernels are persistent (grid = a few workgroups per CU, looping
// over work items) so empty M-slots cost nothing, and each wave keeps D K-blocks of loads in
// flight in a register ring.
//
// GEMM1 item = (M-tile, 16 columns of C). The four waves of a workgroup split the K range
// (H/128 blocks) into quarters, each streaming its quarter of the 16 X1 rows and 16 X2 rows of
// W13; the partial accumulators meet in LDS and wave 0 applies SwiGLU and stores bf16 C.
//
// GEMM2 item = (M-tile, 16 columns of H), one wave per item over the full K = I, with no
// workgroup-level synchronisation. The epilogue scales by the pair's routing weight and stores
// fp32 rows for the combine.
//
// MFMA operand maps and block-scale application are those of moe_gemm.hip.
#include "moe_device.h"
#include "moe_kernels.h"

namespace jgmoe {

template <int MT>
struct S1Stage {
  v8i a[MT];
  v8i b1, b2;
  float sw1, sw2;
};

#ifndef JG_G1S_OCC
#define JG_G1S_OCC
#endif
#ifndef JG_G2S_OCC
#define JG_G2S_OCC
#endif

// Max K blocks (H/128) the activation-scale staging in LDS holds: H <= 16384.
constexpr int kMaxKB = 128;

template <int MT, int D>
__global__ __launch_bounds__(256) JG_G1S_OCC void gemm1_stream_kernel(
    const uint8_t* __restrict__ hs, const float* __restrict__ hs_scale,
    const uint8_t* __restrict__ w13, const float* __restrict__ s13,
    const int32_t* __restrict__ counts, const int32_t* __restrict__ offsets,
    const int32_t* __restrict__ sorted_tok, uint16_t* __restrict__ C, int T, int H, int I,
    int E_l) {
  constexpr int BM = 16 * MT;
  __shared__ float red[3][MT * 8][kWave];
  __shared__ float4 sa_lds[kMaxKB][BM / 4];  // activation scales of the tile rows, [kb][row]
  __shared__ int tok_lds[BM];
  const int lane = threadIdx.x & (kWave - 1), wave = wave_id();
  const int r16 = lane & 15, g = lane >> 4;
  const int NCT = I / 16, NKB = H / kBlock;
  const int kb0 = (NKB * wave) / 4, kb1 = (NKB * (wave + 1)) / 4;
  TileMap tm;
  tm.init(counts, offsets, E_l, BM);
  const int items = tm.total * NCT;
  const __amdgpu_buffer_rsrc_t ares = make_rsrc(hs, (uint32_t)T * H);
  int prev_tile = -1;

  for (int item = blockIdx.x; item < items; item += gridDim.x) {
    const int tile = item / NCT, ct = item % NCT;
    int m0, cnt, seg;
    const int e = tm.find(tile, BM, m0, cnt, seg);
    const int c0 = ct * 16;
    // Buffer loads: SGPR resource + one VGPR lane offset + SGPR K offset per load.
    const __amdgpu_buffer_rsrc_t wres = make_rsrc(w13 + (size_t)e * 2 * I * H, 2u * I * H);
    const uint32_t woff = r16 * H + 32 * g;
    const uint32_t wsoff1 = (uint32_t)c0 * H, wsoff2 = (uint32_t)(I + c0) * H;
    LaneScales sc1, sc2;
    sc1.load(s13 + ((size_t)e * (2 * I / kBlock) + c0 / kBlock) * NKB, NKB);
    sc2.load(s13 + ((size_t)e * (2 * I / kBlock) + (I + c0) / kBlock) * NKB, NKB);

    // Weight loads of the first D K-blocks go out before the tile set-up below, which waits on
    // dependent global reads (token ids, then their scales).
    S1Stage<MT> st[D];
    auto load_b = [&](int kb, S1Stage<MT>& x) {
      x.b1 = buf_load32(wres, woff, wsoff1 + kb * kBlock);
      x.b2 = buf_load32(wres, woff, wsoff2 + kb * kBlock);
      x.sw1 = sc1.get(kb);
      x.sw2 = sc2.get(kb);
    };
#pragma unroll
    for (int d = 0; d < D; ++d)
      if (kb0 + d < kb1) load_b(kb0 + d, st[d]);

    if (tile != prev_tile) {  // uniform across the workgroup
      prev_tile = tile;
      if (threadIdx.x < BM) {
        const int r = m0 + threadIdx.x;
        tok_lds[threadIdx.x] = r < cnt ? sorted_tok[seg + r] : -1;
      }
      __syncthreads();
      float* sa = (float*)sa_lds;
      for (int i = threadIdx.x; i < NKB * BM; i += blockDim.x) {
        const int tk = tok_lds[i % BM];
        sa[i] = tk >= 0 ? hs_scale[(size_t)(i / BM) * T + tk] : 0.f;
      }
      __syncthreads();
    }

    // Rows past the segment end re-read the last valid row: MFMA output rows depend only on
    // their own A row, and those rows are never stored.
    uint32_t aoff[MT];
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
      const int ri = mt * 16 + r16, last = min(cnt - m0, BM) - 1;
      const int tk = tok_lds[ri <= last ? ri : last];
      aoff[mt] = (uint32_t)tk * H + 32 * g;
    }
    auto load_a = [&](int kb, S1Stage<MT>& x) {
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) x.a[mt] = buf_load32(ares, aoff[mt], kb * kBlock);
    };

    v4f acc1[MT], acc2[MT];
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
      acc1[mt] = v4f{0.f, 0.f, 0.f, 0.f};
      acc2[mt] = v4f{0.f, 0.f, 0.f, 0.f};
    }
    auto compute = [&](int kb, const S1Stage<MT>& x) {
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) {
        const float4 sa = sa_lds[kb][mt * 4 + g];
        const v4f p = mfma_f8_16x16x128(x.a[mt], x.b1);
        const v4f q = mfma_f8_16x16x128(x.a[mt], x.b2);
        acc1[mt][0] = fmaf(p[0], sa.x * x.sw1, acc1[mt][0]);
        acc1[mt][1] = fmaf(p[1], sa.y * x.sw1, acc1[mt][1]);
        acc1[mt][2] = fmaf(p[2], sa.z * x.sw1, acc1[mt][2]);
        acc1[mt][3] = fmaf(p[3], sa.w * x.sw1, acc1[mt][3]);
        acc2[mt][0] = fmaf(q[0], sa.x * x.sw2, acc2[mt][0]);
        acc2[mt][1] = fmaf(q[1], sa.y * x.sw2, acc2[mt][1]);
        acc2[mt][2] = fmaf(q[2], sa.z * x.sw2, acc2[mt][2]);
        acc2[mt][3] = fmaf(q[3], sa.w * x.sw2, acc2[mt][3]);
      }
    };

#pragma unroll
    for (int d = 0; d < D; ++d)
      if (kb0 + d < kb1) load_a(kb0 + d, st[d]);
    for (int kb = kb0; kb < kb1; kb += D) {
#pragma unroll
      for (int d = 0; d < D; ++d) {
        if (kb + d < kb1) {
          compute(kb + d, st[d]);
          if (kb + d + D < kb1) {
            load_b(kb + d + D, st[d]);
            load_a(kb + d + D, st[d]);
          }
        }
      }
    }

    if (wave > 0) {
#pragma unroll
      for (int mt = 0; mt < MT; ++mt)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          red[wave - 1][mt * 8 + i][lane] = acc1[mt][i];
          red[wave - 1][mt * 8 + 4 + i][lane] = acc2[mt][i];
        }
    }
    __syncthreads();
    if (wave == 0) {
#pragma unroll
      for (int mt = 0; mt < MT; ++mt)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          float x1 = acc1[mt][i], x2 = acc2[mt][i];
#pragma unroll
          for (int w = 0; w < 3; ++w) {
            x1 += red[w][mt * 8 + i][lane];
            x2 += red[w][mt * 8 + 4 + i][lane];
          }
          const int r = m0 + mt * 16 + 4 * g + i;
          if (r < cnt)
            C[(size_t)(seg + r) * I + c0 + r16] =
                float_to_bf16_bits(x1 * (x2 / (1.0f + __expf(-x2))));
        }
    }
    __syncthreads();
  }
}

template <int MT>
struct S2Stage {
  uint4 a[MT][4];
  v8i b;
  float sw;
};

template <int MT, int D>
__global__ __launch_bounds__(256) JG_G2S_OCC void gemm2_stream_kernel(
    const uint16_t* __restrict__ C, const uint8_t* __restrict__ w2, const float* __restrict__ s2,
    const int32_t* __restrict__ counts, const int32_t* __restrict__ offsets,
    const float* __restrict__ sorted_w, float* __restrict__ partial, int H, int I, int E_l,
    int max_pairs) {
  constexpr int BM = 16 * MT;
  const int lane = threadIdx.x & (kWave - 1);
  const __amdgpu_buffer_rsrc_t cres = make_rsrc(C, (uint32_t)max_pairs * I * 2);
  const int r16 = lane & 15, g = lane >> 4;
  const int NHT = H / 16, NKB = I / kBlock;
  TileMap tm;
  tm.init(counts, offsets, E_l, BM);
  const int items = tm.total * NHT;
  const int stride = gridDim.x * (blockDim.x / kWave);

  const int first = blockIdx.x * (blockDim.x / kWave) + wave_id();
  for (int item = first; item < items; item += stride) {
    const int tile = item / NHT, ht = item % NHT;
    int m0, cnt, seg;
    const int e = tm.find(tile, BM, m0, cnt, seg);
    const int h0 = ht * 16;

    uint32_t coff[MT];
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
      const int r = m0 + mt * 16 + r16;
      coff[mt] = ((uint32_t)(seg + (r < cnt ? r : cnt - 1)) * I + 32 * g) * 2;
    }
    const __amdgpu_buffer_rsrc_t wres = make_rsrc(w2 + (size_t)e * H * I, (uint32_t)H * I);
    const uint32_t woff = r16 * I + 32 * g, wsoff = (uint32_t)h0 * I;
    LaneScales sc;
    sc.load(s2 + ((size_t)e * (H / kBlock) + h0 / kBlock) * NKB, NKB);

    v4f acc[MT];
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) acc[mt] = v4f{0.f, 0.f, 0.f, 0.f};

    auto load = [&](int kb, S2Stage<MT>& st) {
      st.b = buf_load32(wres, woff, wsoff + kb * kBlock);
#pragma unroll
      for (int mt = 0; mt < MT; ++mt)
#pragma unroll
        for (int c = 0; c < 4; ++c) st.a[mt][c] = buf_load16(cres, coff[mt], 2 * (kb * kBlock + 8 * c));
      st.sw = sc.get(kb);
    };
    auto compute = [&](const S2Stage<MT>& st) {
      v8bf bc[4];
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        v2bf p0, p1, p2, p3;
        fp8x4_to_bf16x4(st.b[2 * c], p0, p1);
        fp8x4_to_bf16x4(st.b[2 * c + 1], p2, p3);
        bc[c] = v8bf{p0[0], p0[1], p1[0], p1[1], p2[0], p2[1], p3[0], p3[1]};
      }
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) {
        v4f t = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int c = 0; c < 4; ++c)
          t = mfma_bf16_16x16x32(__builtin_bit_cast(v8bf, st.a[mt][c]), bc[c], t);
#pragma unroll
        for (int i = 0; i < 4; ++i) acc[mt][i] = fmaf(t[i], st.sw, acc[mt][i]);
      }
    };

    S2Stage<MT> st[D];
#pragma unroll
    for (int d = 0; d < D; ++d)
      if (d < NKB) load(d, st[d]);
    for (int kb = 0; kb < NKB; kb += D) {
#pragma unroll
      for (int d = 0; d < D; ++d) {
        if (kb + d < NKB) {
          compute(st[d]);
          if (kb + d + D < NKB) load(kb + d + D, st[d]);
        }
      }
    }

#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int r = m0 + mt * 16 + 4 * g + i;
        if (r < cnt) {
          const int p = seg + r;
          partial[(size_t)p * H + h0 + r16] = acc[mt][i] * sorted_w[p];
        }
      }
  }
}

// Persistent grid: `per_cu` workgroups per CU, capped by the largest possible item count.
static int persistent_grid(int per_cu, long long max_items) {
  static int cus = 0;
  if (cus == 0) {
    int dev = 0, n = 0;
    if (hipGetDevice(&dev) == hipSuccess &&
        hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) == hipSuccess && n > 0)
      cus = n;
    else
      cus = 256;
  }
  long long g = (long long)cus * per_cu;
  if (g > max_items) g = max_items;
  return g < 1 ? 1 : (int)g;
}

static inline long long max_m_tiles(int max_pairs, int bm, int E_l) {
  return (max_pairs + bm - 1) / bm + (E_l < max_pairs ? E_l : max_pairs);
}

#ifndef JG_G1_STREAM_D
#define JG_G1_STREAM_D 4
#endif
#ifndef JG_G2_STREAM_D
#define JG_G2_STREAM_D 4
#endif
#ifndef JG_STREAM_PER_CU
#define JG_STREAM_PER_CU 4
#endif

hipError_t launch_gemm1_stream(const uint8_t* hs, const float* hs_scale, const uint8_t* w13,
                               const float* s13, const int32_t* counts, const int32_t* offsets,
                               const int32_t* sorted_tok, uint16_t* C, int T, int H, int I,
                               int E_l, int max_pairs, int mt, hipStream_t stream) {
#define JG_G1S(MT, D)                                                                        \
  {                                                                                          \
    const int grid =                                                                         \
        persistent_grid(JG_STREAM_PER_CU, max_m_tiles(max_pairs, 16 * MT, E_l) * (I / 16));  \
    gemm1_stream_kernel<MT, D><<<grid, 256, 0, stream>>>(hs, hs_scale, w13, s13, counts,     \
                                                         offsets, sorted_tok, C, T, H, I, E_l); \
  }
  if (mt == 1) JG_G1S(1, JG_G1_STREAM_D)
  else if (mt == 2) JG_G1S(2, 3)
  else JG_G1S(4, 2)
#undef JG_G1S
  return hipGetLastError();
}

hipError_t launch_gemm2_stream(const uint16_t* C, const uint8_t* w2, const float* s2,
                               const int32_t* counts, const int32_t* offsets,
                               const float* sorted_w, float* partial, int H, int I, int E_l,
                               int max_pairs, int mt, hipStream_t stream) {
#define JG_G2S(MT, D)                                                                        \
  {                                                                                          \
    const long long waves = max_m_tiles(max_pairs, 16 * MT, E_l) * (H / 16);                 \
    const int grid = persistent_grid(JG_STREAM_PER_CU, (waves + 3) / 4);                     \
    gemm2_stream_kernel<MT, D><<<grid, 256, 0, stream>>>(C, w2, s2, counts, offsets,         \
                                                         sorted_w, partial, H, I, E_l, max_pairs); \
  }
  if (mt == 1) JG_G2S(1, JG_G2_STREAM_D)
  else if (mt == 2) JG_G2S(2, 2)
  else JG_G2S(4, 2)
#undef JG_G2S
  return hipGetLastError();
}

}  // namespace jgmoe
