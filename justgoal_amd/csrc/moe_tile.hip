// LDS-tiled grouped GEMMs for segments of tens to thousands of pairs per expert.
//
// A workgroup computes a BM x (64*NW) tile of one expert's output (BM = 16*MT pairs). The
// activation rows of the tile (fp8 hidden states for GEMM1, bf16 C for GEMM2) change with K only,
// so they are staged once per 128-wide K block in LDS (double buffered, one barrier per K block)
// and shared by the four waves; each wave owns 16*NW output columns and streams its weight rows
// straight from HBM into registers through a D-deep ring of buffer loads. Every weight fragment
// feeds MT MFMAs, every LDS activation fragment feeds 2*NW (GEMM1) or NW (GEMM2) MFMAs.
//
// LDS rows are XOR-swizzled in 16-byte chunks (chunk ^ row) so the 16 rows an MFMA operand read
// touches fall into distinct banks.
//
// Block-scale handling and the K-permutation of the bf16 MFMA are those of moe_gemm.hip.
// Persistent grid; items are (M-tile, N-tile) with the N-tile fastest.
#include "moe_device.h"
#include "moe_kernels.h"

// K-order rotation per work item (0 = off): item i walks K blocks starting at
// (i * JG_TILE_ROT) mod (K/128), so concurrent items read different column ranges.
#ifndef JG_TILE_ROT
#define JG_TILE_ROT 0
#endif
#ifndef JG_G1T_OCC
#define JG_G1T_OCC
#endif
#ifndef JG_G2T_OCC
#define JG_G2T_OCC
#endif

namespace jgmoe {

namespace {

// Per-thread share of an A tile: BM rows x 128 bytes = BM*8 chunks of 16 B over 256 threads.
template <int MT>
struct AStage1 {
  uint4 v[MT / 2 > 0 ? MT / 2 : 1];
};

template <int NW>
struct BStage1 {
  v8i b1[NW], b2[NW];
  float sw1, sw2;
};

}  // namespace

template <int MT, int NW, int D>
__global__ __launch_bounds__(256) JG_G1T_OCC void gemm1_tile_kernel(
    const uint8_t* __restrict__ hs, const float* __restrict__ hs_scale,
    const uint8_t* __restrict__ w13, const float* __restrict__ s13,
    const int32_t* __restrict__ counts, const int32_t* __restrict__ offsets,
    const int32_t* __restrict__ sorted_tok, uint16_t* __restrict__ C, int T, int H, int I,
    int E_l) {
  static_assert(MT % 2 == 0, "A staging assumes an even number of 16-row sub-tiles");
  constexpr int BM = 16 * MT;
  constexpr int ACH = MT / 2;  // 16-byte chunks per thread per K block
  __shared__ __attribute__((aligned(16))) uint8_t a_lds[2][BM * 128];
  __shared__ __attribute__((aligned(16))) float sa_lds[2][256];  // rows >= BM unused
  __shared__ int tok_lds[BM];

  const int tid = threadIdx.x, lane = tid & (kWave - 1), wave = wave_id();
  const int r16 = lane & 15, g = lane >> 4;
  const int NNT = I / (64 * NW), NKB = H / kBlock;
  TileMap tm;
  tm.init(counts, offsets, E_l, BM);
  const int items = tm.total * NNT;
  const __amdgpu_buffer_rsrc_t ares = make_rsrc(hs, (uint32_t)T * H);
  const __amdgpu_buffer_rsrc_t sres = make_rsrc(hs_scale, (uint32_t)T * (H / kBlock) * 4);

  // this thread's A staging chunks: row = (tid + 256*c) / 8, 16-byte chunk = tid % 8
  const int a_chunk = tid & 7;

  for (int item = blockIdx.x; item < items; item += gridDim.x) {
    const int tile = item / NNT, nt = item % NNT;
    int m0, cnt, seg;
    const int e = tm.find(tile, BM, m0, cnt, seg);
    const int c0 = nt * 64 * NW + wave * 16 * NW;
    const int rot = (item * JG_TILE_ROT) % NKB;
    // K-block index of loop step kb; steps past the end map onto the last step's block.
    auto kmap = [&](int kb) {
      kb = min(kb, NKB - 1) + rot;
      return kb >= NKB ? kb - NKB : kb;
    };

    const __amdgpu_buffer_rsrc_t wres = make_rsrc(w13 + (size_t)e * 2 * I * H, 2u * I * H);
    const uint32_t woff = r16 * H + 32 * g;
    const uint32_t ws1 = (uint32_t)c0 * H, ws2 = (uint32_t)(I + c0) * H;
    LaneScales sc1, sc2;
    sc1.load(s13 + ((size_t)e * (2 * I / kBlock) + c0 / kBlock) * NKB, NKB);
    sc2.load(s13 + ((size_t)e * (2 * I / kBlock) + (I + c0) / kBlock) * NKB, NKB);

    BStage1<NW> bst[D];
    auto load_b = [&](int kb, BStage1<NW>& x) {
      kb = kmap(kb);  // prefetches past the end re-read the last block, never used
#pragma unroll
      for (int j = 0; j < NW; ++j) {
        x.b1[j] = buf_load32(wres, woff, ws1 + (uint32_t)j * 16 * H + kb * kBlock);
        x.b2[j] = buf_load32(wres, woff, ws2 + (uint32_t)j * 16 * H + kb * kBlock);
      }
      x.sw1 = sc1.get(kb);
      x.sw2 = sc2.get(kb);
    };
#pragma unroll
    for (int d = 0; d < D; ++d) load_b(d, bst[d]);

    __syncthreads();  // previous item's readers of tok_lds / a_lds are done
    if (tid < BM) {
      const int r = m0 + tid;
      tok_lds[tid] = sorted_tok[seg + (r < cnt ? r : cnt - 1)];
    }
    __syncthreads();
    uint32_t aoff[ACH];
#pragma unroll
    for (int c = 0; c < ACH; ++c) aoff[c] = (uint32_t)tok_lds[(tid + 256 * c) / 8] * H + 16 * a_chunk;
    const int sa_tok = tid < BM ? tok_lds[tid] : 0;

    // A ring: slot d holds the activation chunks (and this row's scale) of a K block kb with
    // kb % D == d, loaded D blocks ahead of its compute.
    AStage1<MT> ast[D];
    float sa_next[D];
    auto load_a = [&](int kb, int slot_unused, AStage1<MT>& x, float& sx) {
      (void)slot_unused;
      kb = kmap(kb);
#pragma unroll
      for (int c = 0; c < ACH; ++c) x.v[c] = buf_load16(ares, aoff[c], kb * kBlock);
      // every thread loads (rows past BM re-read row 0) so the load count per stage is uniform
      sx = __uint_as_float(buf_load32b(sres, (uint32_t)sa_tok * 4, (uint32_t)kb * T * 4));
    };
    auto store_a = [&](int buf, const AStage1<MT>& x, float sx) {
#pragma unroll
      for (int c = 0; c < ACH; ++c) {
        const int row = (tid + 256 * c) / 8;
        *(uint4*)&a_lds[buf][row * 128 + ((a_chunk ^ (row & 7)) * 16)] = x.v[c];
      }
      sa_lds[buf][tid] = sx;  // unconditional: no divergent branch in the K loop
    };

    v4f acc1[MT][NW], acc2[MT][NW];
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
      for (int j = 0; j < NW; ++j) {
        acc1[mt][j] = v4f{0.f, 0.f, 0.f, 0.f};
        acc2[mt][j] = v4f{0.f, 0.f, 0.f, 0.f};
      }

    // Weights go in as the MFMA's first operand, so lane l holds output row (l & 15) and the
    // four columns 4*(l>>4)+i: the activation scale is then one value per lane and K block.
    auto compute = [&](int buf, const BStage1<NW>& x) {
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) {
        const int row = mt * 16 + r16;
        const uint4 lo = *(const uint4*)&a_lds[buf][row * 128 + (((2 * g) ^ (row & 7)) * 16)];
        const uint4 hi = *(const uint4*)&a_lds[buf][row * 128 + (((2 * g + 1) ^ (row & 7)) * 16)];
        const v8i a = v8i{(int)lo.x, (int)lo.y, (int)lo.z, (int)lo.w,
                          (int)hi.x, (int)hi.y, (int)hi.z, (int)hi.w};
        const float sa = sa_lds[buf][row];
        const float f1 = sa * x.sw1, f2 = sa * x.sw2;
#pragma unroll
        for (int j = 0; j < NW; ++j) {
          const v4f p = mfma_f8_16x16x128(x.b1[j], a);
          const v4f q = mfma_f8_16x16x128(x.b2[j], a);
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            acc1[mt][j][i] = fmaf(p[i], f1, acc1[mt][j][i]);
            acc2[mt][j][i] = fmaf(q[i], f2, acc2[mt][j][i]);
          }
        }
      }
    };

#pragma unroll
    for (int d = 0; d < D; ++d) load_a(d, d, ast[d], sa_next[d]);
    store_a(0, ast[0], sa_next[0]);
    load_a(D, 0, ast[0], sa_next[0]);
    __syncthreads();
    // One K block: compute from LDS buffer kb&1, prefetch block kb+D into the B ring, move
    // block kb+1 from the A ring into the other LDS buffer and prefetch block kb+1+D into the
    // A ring. Prefetch indices are clamped, so the step has no branches.
    auto step = [&](int d, int kb) {
      compute(kb & 1, bst[d]);
      // Scheduling fences keep each prefetch where it is written: without them the scheduler
      // sinks the loads next to their use and every K block waits on memory.
      __builtin_amdgcn_sched_barrier(0);
      load_b(kb + D, bst[d]);
      __builtin_amdgcn_sched_barrier(0);
      const int dn = (d + 1) % D;  // compile-time after unrolling
      store_a((kb + 1) & 1, ast[dn], sa_next[dn]);
      load_a(kb + 1 + D, dn, ast[dn], sa_next[dn]);
      __builtin_amdgcn_sched_barrier(0);
      __syncthreads();
    };
    // Whole trips of D blocks run without conditionals (a conditional load inside the loop
    // makes the compiler wait for every outstanding load at each trip); the remainder runs
    // after the loop.
    const int nfull = NKB / D * D;
    for (int kb0 = 0; kb0 < nfull; kb0 += D) {
#pragma unroll
      for (int d = 0; d < D; ++d) step(d, kb0 + d);
    }
#pragma unroll
    for (int d = 0; d < D - 1; ++d)
      if (nfull + d < NKB) step(d, nfull + d);

#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
      const int r = m0 + mt * 16 + r16;
      if (r < cnt) {
        uint16_t* crow = C + (size_t)(seg + r) * I + c0 + 4 * g;
#pragma unroll
        for (int j = 0; j < NW; ++j) {
          uint32_t h[4];
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const float x1 = acc1[mt][j][i], x2 = acc2[mt][j][i];
            h[i] = float_to_bf16_bits(x1 * (x2 / (1.0f + __expf(-x2))));
          }
          *(uint2*)(crow + 16 * j) = uint2{h[0] | (h[1] << 16), h[2] | (h[3] << 16)};
        }
      }
    }
  }
}

namespace {

template <int MT>
struct AStage2 {
  uint4 v[MT];  // BM rows x 256 bytes = BM*16 chunks over 256 threads
};

template <int NW>
struct BStage2 {
  v8i b[NW];
  float sw;
};

}  // namespace

template <int MT, int NW, int D>
__global__ __launch_bounds__(256) JG_G2T_OCC void gemm2_tile_kernel(
    const uint16_t* __restrict__ C, const uint8_t* __restrict__ w2, const float* __restrict__ s2,
    const int32_t* __restrict__ counts, const int32_t* __restrict__ offsets,
    const float* __restrict__ sorted_w, float* __restrict__ partial, int H, int I, int E_l,
    int max_pairs) {
  constexpr int BM = 16 * MT;
  __shared__ __attribute__((aligned(16))) uint8_t a_lds[2][BM * 256];

  const int tid = threadIdx.x, lane = tid & (kWave - 1), wave = wave_id();
  const int r16 = lane & 15, g = lane >> 4;
  const int NNT = H / (64 * NW), NKB = I / kBlock;
  TileMap tm;
  tm.init(counts, offsets, E_l, BM);
  const int items = tm.total * NNT;
  const __amdgpu_buffer_rsrc_t cres = make_rsrc(C, (uint32_t)max_pairs * I * 2);
  const int a_chunk = tid & 15;

  for (int item = blockIdx.x; item < items; item += gridDim.x) {
    const int tile = item / NNT, nt = item % NNT;
    int m0, cnt, seg;
    const int e = tm.find(tile, BM, m0, cnt, seg);
    const int h0 = nt * 64 * NW + wave * 16 * NW;
    const int rot = (item * JG_TILE_ROT) % NKB;
    auto kmap = [&](int kb) {
      kb = min(kb, NKB - 1) + rot;
      return kb >= NKB ? kb - NKB : kb;
    };

    const __amdgpu_buffer_rsrc_t wres = make_rsrc(w2 + (size_t)e * H * I, (uint32_t)H * I);
    const uint32_t woff = r16 * I + 32 * g, wsoff = (uint32_t)h0 * I;
    LaneScales sc;
    sc.load(s2 + ((size_t)e * (H / kBlock) + h0 / kBlock) * NKB, NKB);

    BStage2<NW> bst[D];
    auto load_b = [&](int kb, BStage2<NW>& x) {
      kb = kmap(kb);  // prefetches past the end re-read the last block, never used
#pragma unroll
      for (int j = 0; j < NW; ++j)
        x.b[j] = buf_load32(wres, woff, wsoff + (uint32_t)j * 16 * I + kb * kBlock);
      x.sw = sc.get(kb);
    };
#pragma unroll
    for (int d = 0; d < D; ++d) load_b(d, bst[d]);

    uint32_t aoff[MT];
#pragma unroll
    for (int c = 0; c < MT; ++c) {
      const int row = (tid + 256 * c) / 16;
      const int r = m0 + row;
      aoff[c] = ((uint32_t)(seg + (r < cnt ? r : cnt - 1)) * I) * 2 + 16 * a_chunk;
    }
    AStage2<MT> ast[D];
    auto load_a = [&](int kb, AStage2<MT>& x) {
      kb = kmap(kb);
#pragma unroll
      for (int c = 0; c < MT; ++c) x.v[c] = buf_load16(cres, aoff[c], kb * kBlock * 2);
    };
    auto store_a = [&](int buf, const AStage2<MT>& x) {
#pragma unroll
      for (int c = 0; c < MT; ++c) {
        const int row = (tid + 256 * c) / 16;
        *(uint4*)&a_lds[buf][row * 256 + ((a_chunk ^ (row & 15)) * 16)] = x.v[c];
      }
    };

    v4f acc[MT][NW];
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
      for (int j = 0; j < NW; ++j) acc[mt][j] = v4f{0.f, 0.f, 0.f, 0.f};

    auto compute = [&](int buf, const BStage2<NW>& x) {
      v8bf bc[NW][4];
#pragma unroll
      for (int j = 0; j < NW; ++j)
#pragma unroll
        for (int c = 0; c < 4; ++c) {
          v2bf p0, p1, p2, p3;
          fp8x4_to_bf16x4(x.b[j][2 * c], p0, p1);
          fp8x4_to_bf16x4(x.b[j][2 * c + 1], p2, p3);
          bc[j][c] = v8bf{p0[0], p0[1], p1[0], p1[1], p2[0], p2[1], p3[0], p3[1]};
        }
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) {
        const int row = mt * 16 + r16;
        v8bf a[4];
#pragma unroll
        for (int c = 0; c < 4; ++c)
          a[c] = __builtin_bit_cast(
              v8bf, *(const uint4*)&a_lds[buf][row * 256 + (((4 * g + c) ^ (row & 15)) * 16)]);
#pragma unroll
        for (int j = 0; j < NW; ++j) {
          v4f t = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
          for (int c = 0; c < 4; ++c) t = mfma_bf16_16x16x32(a[c], bc[j][c], t);
#pragma unroll
          for (int i = 0; i < 4; ++i) acc[mt][j][i] = fmaf(t[i], x.sw, acc[mt][j][i]);
        }
      }
    };

#pragma unroll
    for (int d = 0; d < D; ++d) load_a(d, ast[d]);
    __syncthreads();  // previous item's LDS readers are done
    store_a(0, ast[0]);
    load_a(D, ast[0]);
    __syncthreads();
    // Same K-block step and loop split as the GEMM1 tile kernel.
    auto step = [&](int d, int kb) {
      compute(kb & 1, bst[d]);
      __builtin_amdgcn_sched_barrier(0);
      load_b(kb + D, bst[d]);
      __builtin_amdgcn_sched_barrier(0);
      const int dn = (d + 1) % D;
      store_a((kb + 1) & 1, ast[dn]);
      load_a(kb + 1 + D, ast[dn]);
      __builtin_amdgcn_sched_barrier(0);
      __syncthreads();
    };
    const int nfull = NKB / D * D;
    for (int kb0 = 0; kb0 < nfull; kb0 += D) {
#pragma unroll
      for (int d = 0; d < D; ++d) step(d, kb0 + d);
    }
#pragma unroll
    for (int d = 0; d < D - 1; ++d)
      if (nfull + d < NKB) step(d, nfull + d);

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
}

static int tile_grid(int per_cu, long long max_items) {
  static int cus = 0;
  if (cus == 0) {
    int dev = 0, n = 0;
    cus = (hipGetDevice(&dev) == hipSuccess &&
           hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) == hipSuccess &&
           n > 0)
              ? n
              : 256;
  }
  long long g = (long long)cus * per_cu;
  if (g > max_items) g = max_items;
  return g < 1 ? 1 : (int)g;
}

#ifndef JG_TILE_PER_CU
#define JG_TILE_PER_CU 2
#endif
#ifndef JG_G1T_NW
#define JG_G1T_NW 1
#endif
#ifndef JG_G2T_NW
#define JG_G2T_NW 2
#endif
#ifndef JG_TILE_D
#define JG_TILE_D 2
#endif

hipError_t launch_gemm1_tile(const uint8_t* hs, const float* hs_scale, const uint8_t* w13,
                             const float* s13, const int32_t* counts, const int32_t* offsets,
                             const int32_t* sorted_tok, uint16_t* C, int T, int H, int I, int E_l,
                             int max_pairs, int mt, hipStream_t stream) {
#define JG_G1T(MT, NW)                                                                        \
  {                                                                                           \
    const long long tiles = (max_pairs + 16 * MT - 1) / (16 * MT) + (E_l < max_pairs ? E_l : max_pairs); \
    const int grid = tile_grid(JG_TILE_PER_CU, tiles * (I / (64 * NW)));                      \
    gemm1_tile_kernel<MT, NW, JG_TILE_D><<<grid, 256, 0, stream>>>(                           \
        hs, hs_scale, w13, s13, counts, offsets, sorted_tok, C, T, H, I, E_l);                \
  }
  if (mt <= 2) JG_G1T(2, JG_G1T_NW)
  else if (mt <= 4) JG_G1T(4, JG_G1T_NW)
  else JG_G1T(8, JG_G1T_NW)
#undef JG_G1T
  return hipGetLastError();
}

hipError_t launch_gemm2_tile(const uint16_t* C, const uint8_t* w2, const float* s2,
                             const int32_t* counts, const int32_t* offsets,
                             const float* sorted_w, float* partial, int H, int I, int E_l,
                             int max_pairs, int mt, hipStream_t stream) {
#define JG_G2T(MT, NW)                                                                        \
  {                                                                                           \
    const long long tiles = (max_pairs + 16 * MT - 1) / (16 * MT) + (E_l < max_pairs ? E_l : max_pairs); \
    const int grid = tile_grid(JG_TILE_PER_CU, tiles * (H / (64 * NW)));                      \
    gemm2_tile_kernel<MT, NW, JG_TILE_D><<<grid, 256, 0, stream>>>(                           \
        C, w2, s2, counts, offsets, sorted_w, partial, H, I, E_l, max_pairs);                 \
  }
  if (mt <= 2) JG_G2T(2, JG_G2T_NW)
  else if (mt <= 4) JG_G2T(4, JG_G2T_NW)
  else JG_G2T(8, JG_G2T_NW)
#undef JG_G2T
  return hipGetLastError();
}

}  // namespace jgmoe
