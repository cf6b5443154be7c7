// Large-tile grouped GEMMs for long per-expert segments (prefill-sized batches).
//
// A workgroup of four waves in a 2x2 grid computes a BM x BN output tile of one expert: each wave
// owns (BM/2) x (BN/2). Both operands reach LDS by DMA into rings of D slots shared by the four
// waves, so every weight K-block is fetched once per BM rows (not once per 16 columns per wave as
// in the smaller tiles) and every activation K-block once per BN columns:
//
// * GEMM1: BM rows of fp8 hidden states (gathered from the token rows) plus their activation
//   scales, and BN columns of C, i.e. BN X1 rows and BN X2 rows of W13. The epilogue applies
//   SwiGLU and stores bf16 C.
// * GEMM2: BM rows of bf16 C and BN rows of W2; the epilogue scales by the pair's routing weight
//   and stores fp32 rows for the combine.
//
// Per K step: each wave waits for its own DMAs of the step's block (counted vmcnt), one bare
// s_barrier makes all of them visible and frees the slot read in the previous step, the slot is
// refilled with the block D-1 steps ahead (across item boundaries; the next item's per-lane
// metadata arrives by 4-byte DMA in a per-wave LDS area), then the wave reads its MFMA fragments
// from LDS and runs (BM/32)*(BN/32) fragment products per matrix. LDS images use the XOR chunk
// swizzle of the other kernels; MFMA forms and scale handling are those of moe_tile.hip.
#include "moe_device.h"
#include "moe_kernels.h"

namespace jgmoe {

namespace {

constexpr int kWaves = 4;
constexpr int kWBlk = 16 * kBlock;  // 16 rows x 128 bytes

constexpr int vm_depth(int n) { return n > 63 ? 63 : n < 0 ? 0 : n; }

// ---- GEMM1 ------------------------------------------------------------------------------------
//
// Five waves: waves 0..3 compute (2x2 grid over the BM x BN tile), wave 4 is the producer that
// issues every DMA of the workgroup and waits on their counts. A wave stalled issuing DMAs (the
// CU's texture path takes about 70 cycles per 1 KiB instruction under load) cannot issue MFMAs,
// so keeping the two roles in different waves lets the DMA stream, the LDS reads and the MFMAs
// overlap. Per K step every wave passes one barrier: the producer after its DMAs of the step's
// block have landed (then it refills the slot freed by the previous step), the compute waves
// before reading the block.

constexpr int kComputeWaves = 4;
constexpr int kProducer = 4;  // wave index of the producer

struct B1Scalars {
  const uint8_t* wbase;  // the expert's W13
  uint32_t c0;           // first C column of the tile
  int e, m0, cnt, seg;
};

// MS: 16-row sub-tiles per compute wave (BM = 32*MS); NS: 16-column sub-tiles (BN = 32*NS).
template <int MS, int NS, int D>
__global__ __launch_bounds__(320) void gemm1_big_kernel(
    const uint8_t* __restrict__ hs, const float* __restrict__ hs_scale,
    const uint8_t* __restrict__ w13, const float* __restrict__ s13,
    const int32_t* __restrict__ counts, const int32_t* __restrict__ offsets,
    const int32_t* __restrict__ sorted_tok, uint16_t* __restrict__ C, int T, int H, int I,
    int E_l, int max_pairs) {
  static_assert(D >= 3, "the prefetch lead is D-1 blocks");
  static_assert(16 * NS <= kBlock && kBlock % (16 * NS) == 0, "a wave's columns share one scale block");
  constexpr int BM = 32 * MS, BN = 32 * NS;
  constexpr int AI = BM / 8;        // A DMA instructions per step (8 rows x 128 B each)
  constexpr int SI = BM / 64;       // activation-scale DMA instructions per step
  constexpr int BI = 2 * BN / 8;    // B DMA instructions per step
  constexpr int OPS = AI + SI + BI; // producer vector-memory operations per step
  constexpr int ASZ = BM * kBlock, BSZ = 2 * BN * kBlock;
  __shared__ __attribute__((aligned(16))) uint8_t aring[D][ASZ];
  __shared__ __attribute__((aligned(16))) uint8_t bring[D][BSZ];
  __shared__ __attribute__((aligned(16))) float sring[D][BM];
  __shared__ __attribute__((aligned(16))) int32_t tokl[BM];              // producer: next tile's tokens
  __shared__ __attribute__((aligned(16))) float mring[kComputeWaves][4][kWave];  // weight-scale rows

  const int lane = threadIdx.x & (kWave - 1), w = wave_id();
  const int NNT = I / BN, NKB = H / kBlock;
  TileMap tm;
  tm.init(counts, offsets, E_l, BM);
  const int items = tm.total * NNT;
  int it = uniform((int)blockIdx.x);
  if (it >= items) return;  // whole workgroup
  const int stride = gridDim.x;

  auto scalars = [&](int item, B1Scalars& x) {
    item = uniform(item);
    const int tile = item / NNT, nt = item % NNT;
    x.e = uniform(tm.find(tile, BM, x.m0, x.cnt, x.seg));
    x.m0 = uniform(x.m0);
    x.cnt = uniform(x.cnt);
    x.seg = uniform(x.seg);
    x.c0 = uniform((uint32_t)(nt * BN));
    x.wbase = uniform(w13 + (size_t)x.e * 2 * I * H);
  };
  int it_n = it + stride;

  if (w == kProducer) {
    // ---------------- producer ----------------
    const __amdgpu_buffer_rsrc_t ares = make_rsrc(hs, (uint32_t)T * H);
    const __amdgpu_buffer_rsrc_t sares = make_rsrc(hs_scale, (uint32_t)T * NKB * 4);
    const __amdgpu_buffer_rsrc_t tokres = make_rsrc(sorted_tok, (uint32_t)max_pairs * 4);
    const uint32_t dma0 = wblk_dma_off(lane, 0, H), dma1 = wblk_dma_off(lane, 1, H);
    struct P {
      B1Scalars s;
      uint32_t aoff[AI], saoff[SI];
    };
    // The tile's token list (clamped to its last row) arrives in tokl by 4-byte DMA ...
    auto meta = [&](int item, P& x) {
      scalars(item, x.s);
      const int last = x.s.cnt - 1;
#pragma unroll
      for (int k = 0; k < BM / kWave; ++k) {
        const int r = x.s.m0 + k * kWave + lane;
        dma4(tokres, &tokl[k * kWave], 4u * (x.s.seg + (r < last ? r : last)), 0);
      }
    };
    // ... and is turned into per-lane DMA offsets once it has landed.
    auto finish = [&](P& x) {
      const uint32_t tb = lds_addr(tokl);
      float t[AI + SI];
#pragma unroll
      for (int j = 0; j < AI; ++j) t[j] = ds_read4f(tb + 4 * (8 * j + (lane >> 3)));
#pragma unroll
      for (int k = 0; k < SI; ++k) t[AI + k] = ds_read4f(tb + 4 * (k * kWave + lane));
      lds_wait_all();
#pragma unroll
      for (int j = 0; j < AI + SI; ++j) lds_fence(t[j]);
#pragma unroll
      for (int j = 0; j < AI; ++j)
        x.aoff[j] = __float_as_uint(t[j]) * H + 16 * ((lane & 7) ^ wblk_swz(8 * j + (lane >> 3)));
#pragma unroll
      for (int k = 0; k < SI; ++k) x.saoff[k] = __float_as_uint(t[AI + k]) * 4;
    };
    P cur, nxt, nn;
    meta(it, cur);
    vm_wait<0>();
    finish(cur);
    meta(it_n < items ? it_n : it, nxt);
    vm_wait<0>();
    finish(nxt);

    auto issue = [&](bool second, int kbi, int slot) {
      const P& x = second ? nxt : cur;
#pragma unroll
      for (int j = 0; j < AI; ++j)
        dma16(ares, &aring[slot][j * 1024], second ? nxt.aoff[j] : cur.aoff[j],
              (uint32_t)kbi * kBlock);
#pragma unroll
      for (int k = 0; k < SI; ++k)
        dma4(sares, &sring[slot][k * kWave], second ? nxt.saoff[k] : cur.saoff[k],
             (uint32_t)kbi * T * 4);
      const __amdgpu_buffer_rsrc_t wres = make_rsrc(uniform(x.s.wbase), 2u * I * H);
      const uint32_t c0 = uniform(x.s.c0);
#pragma unroll
      for (int j = 0; j < BI; ++j) {
        const int grp = j >> 1;
        const uint32_t row0 = grp < BN / 16 ? c0 + 16 * grp : I + c0 + 16 * (grp - BN / 16);
        dma16(wres, &bring[slot][j * 1024], (j & 1) ? dma1 : dma0,
              uniform(row0 * H + (uint32_t)kbi * kBlock));
      }
    };
#pragma unroll
    for (int d = 0; d < D - 1; ++d) {
      issue(false, d, d);
      __builtin_amdgcn_sched_barrier(0);
    }
    int slot = 0;
    for (;;) {
      const int it_nn = it_n + stride;
      meta(it_nn < items ? it_nn : (it_n < items ? it_n : it), nn);
      int kb = 0;
      do {
        vm_wait<vm_depth((D - 2) * OPS)>();  // the DMAs of block kb have landed
        __builtin_amdgcn_s_barrier();
        const int kn = kb + D - 1;
        const bool second = kn >= NKB;
        issue(second, second ? kn - NKB : kn, slot == 0 ? D - 1 : slot - 1);
        __builtin_amdgcn_sched_barrier(0);
        slot = slot + 1 == D ? 0 : slot + 1;
        ++kb;
      } while (kb < NKB);
      vm_wait<vm_depth((D - 1) * OPS)>();  // the token-list DMAs of the next-but-one tile
      finish(nn);
      if (it_n >= items) break;
      it = it_n;
      it_n = it_nn;
      cur = nxt;
      nxt = nn;
    }
    vm_wait<0>();  // no DMA may still target this workgroup's LDS when it retires
    return;
  }

  // ---------------- compute waves ----------------
  const int wm = w & 1, wn = w >> 1;
  const int r16 = lane & 15, g = lane >> 4;
  const __amdgpu_buffer_rsrc_t s13res = make_rsrc(s13, (uint32_t)E_l * (2 * I / kBlock) * NKB * 4);
  const uint32_t rd0 = wblk_read_off(lane, 0), rd1 = wblk_read_off(lane, 1);
  float* my_meta = &mring[w][0][0];
  struct Q {
    B1Scalars s;
    LaneScales sc1, sc2;  // weight scales of this wave's X1 / X2 columns
  };
  auto meta = [&](int item, Q& x) {
    scalars(item, x.s);
    const int wc = x.s.c0 + wn * 16 * NS;
    const uint32_t so1 = uniform((uint32_t)((x.s.e * (2 * I / kBlock) + wc / kBlock) * NKB) * 4);
    const uint32_t so2 =
        uniform((uint32_t)((x.s.e * (2 * I / kBlock) + (I + wc) / kBlock) * NKB) * 4);
    dma4(s13res, my_meta + 0 * kWave, 4u * lane, so1);
    dma4(s13res, my_meta + 1 * kWave, 4u * (lane + kWave), so1);
    dma4(s13res, my_meta + 2 * kWave, 4u * lane, so2);
    dma4(s13res, my_meta + 3 * kWave, 4u * (lane + kWave), so2);
  };
  auto finish = [&](Q& x) {
    const uint32_t mb = lds_addr(my_meta) + 4 * lane;
    float v[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) v[j] = ds_read4f(mb + j * 4 * kWave);
    lds_wait_all();
#pragma unroll
    for (int j = 0; j < 4; ++j) lds_fence(v[j]);
    x.sc1.v0 = v[0];
    x.sc1.v1 = v[1];
    x.sc2.v0 = v[2];
    x.sc2.v1 = v[3];
  };
  Q cur, nxt, nn;
  meta(it, cur);
  vm_wait<0>();
  finish(cur);
  meta(it_n < items ? it_n : it, nxt);
  vm_wait<0>();
  finish(nxt);

  int slot = 0;
  for (;;) {
    const int it_nn = it_n + stride;
    meta(it_nn < items ? it_nn : (it_n < items ? it_n : it), nn);
    v4f acc1[MS][NS], acc2[MS][NS];
#pragma unroll
    for (int ms = 0; ms < MS; ++ms)
#pragma unroll
      for (int ns = 0; ns < NS; ++ns) {
        acc1[ms][ns] = v4f{0.f, 0.f, 0.f, 0.f};
        acc2[ms][ns] = v4f{0.f, 0.f, 0.f, 0.f};
      }
    int kb = 0;
    do {
      const int d = slot;
      __builtin_amdgcn_s_barrier();  // block kb is in slot d; everyone is done with slot d-1
      const uint32_t ab = lds_addr(&aring[d][0]) + wm * MS * kWBlk;
      const uint32_t bb = lds_addr(&bring[d][0]) + wn * NS * kWBlk;
      const uint32_t sb = lds_addr(&sring[d][0]) + 4 * (wm * MS * 16 + r16);
      v4u b1l[NS], b1h[NS], b2l[NS], b2h[NS];
#pragma unroll
      for (int ns = 0; ns < NS; ++ns) {
        b1l[ns] = ds_read16(bb + ns * kWBlk + rd0);
        b1h[ns] = ds_read16(bb + ns * kWBlk + rd1);
        b2l[ns] = ds_read16(bb + (BN / 16 + ns) * kWBlk + rd0);
        b2h[ns] = ds_read16(bb + (BN / 16 + ns) * kWBlk + rd1);
      }
      v4u al = ds_read16(ab + rd0), ah = ds_read16(ab + rd1);
      float sa = ds_read4f(sb);
      const float sw1 = cur.sc1.get(kb), sw2 = cur.sc2.get(kb);
      lds_wait_all();
      v8i b1[NS], b2[NS];
#pragma unroll
      for (int ns = 0; ns < NS; ++ns) {
        lds_fence(b1l[ns]);
        lds_fence(b1h[ns]);
        lds_fence(b2l[ns]);
        lds_fence(b2h[ns]);
        b1[ns] = v8i{(int)b1l[ns][0], (int)b1l[ns][1], (int)b1l[ns][2], (int)b1l[ns][3],
                     (int)b1h[ns][0], (int)b1h[ns][1], (int)b1h[ns][2], (int)b1h[ns][3]};
        b2[ns] = v8i{(int)b2l[ns][0], (int)b2l[ns][1], (int)b2l[ns][2], (int)b2l[ns][3],
                     (int)b2h[ns][0], (int)b2h[ns][1], (int)b2h[ns][2], (int)b2h[ns][3]};
      }
      lds_fence(al);
      lds_fence(ah);
      lds_fence(sa);
      // Software pipeline over the MS sub-tiles: sub-tile ms+1's fragments are read while
      // sub-tile ms runs its MFMAs.
#pragma unroll
      for (int ms = 0; ms < MS; ++ms) {
        const v8i a = v8i{(int)al[0], (int)al[1], (int)al[2], (int)al[3],
                          (int)ah[0], (int)ah[1], (int)ah[2], (int)ah[3]};
        const float f1 = sa * sw1, f2 = sa * sw2;
        if (ms + 1 < MS) {
          al = ds_read16(ab + (ms + 1) * kWBlk + rd0);
          ah = ds_read16(ab + (ms + 1) * kWBlk + rd1);
          sa = ds_read4f(sb + 4 * 16 * (ms + 1));
        }
#pragma unroll
        for (int ns = 0; ns < NS; ++ns) {
          const v4f p = mfma_f8_16x16x128(b1[ns], a);
          const v4f q = mfma_f8_16x16x128(b2[ns], a);
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            acc1[ms][ns][i] = fmaf(p[i], f1, acc1[ms][ns][i]);
            acc2[ms][ns][i] = fmaf(q[i], f2, acc2[ms][ns][i]);
          }
        }
        if (ms + 1 < MS) {
          lds_wait_all();
          lds_fence(al);
          lds_fence(ah);
          lds_fence(sa);
        }
      }
      slot = slot + 1 == D ? 0 : slot + 1;
      ++kb;
    } while (kb < NKB);
    vm_wait<0>();  // only this item's scale-row DMAs (and older stores) are outstanding
    finish(nn);

#pragma unroll
    for (int ms = 0; ms < MS; ++ms) {
      const int r = cur.s.m0 + (wm * MS + ms) * 16 + r16;
      if (r < cur.s.cnt) {
        uint16_t* crow = C + (size_t)(cur.s.seg + r) * I + cur.s.c0 + wn * 16 * NS + 4 * g;
#pragma unroll
        for (int ns = 0; ns < NS; ++ns) {
          uint32_t h[4];
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const float x1 = acc1[ms][ns][i], x2 = acc2[ms][ns][i];
            h[i] = float_to_bf16_bits(x1 * (x2 / (1.0f + __expf(-x2))));
          }
          *(uint2*)(crow + 16 * ns) = uint2{h[0] | (h[1] << 16), h[2] | (h[3] << 16)};
        }
      }
    }
    if (it_n >= items) break;
    it = it_n;
    it_n = it_nn;
    cur = nxt;
    nxt = nn;
  }
}

// ---- GEMM2 ------------------------------------------------------------------------------------
//
// Same roles as GEMM1: wave 4 issues the DMAs (bf16 C rows, W2 rows), waves 0..3 compute.

struct B2Scalars {
  const uint8_t* wbase;  // the expert's W2
  uint32_t h0;           // first H column of the tile
  int e, m0, cnt, seg;
};

template <int MS, int NS, int D>
__global__ __launch_bounds__(320) void gemm2_big_kernel(
    const uint16_t* __restrict__ C, const uint8_t* __restrict__ w2, const float* __restrict__ s2,
    const int32_t* __restrict__ counts, const int32_t* __restrict__ offsets,
    const float* __restrict__ sorted_w, float* __restrict__ partial, int H, int I, int E_l,
    int max_pairs) {
  static_assert(D >= 3, "the prefetch lead is D-1 blocks");
  static_assert(16 * NS <= kBlock && kBlock % (16 * NS) == 0, "a wave's columns share one scale block");
  constexpr int BM = 32 * MS, BN = 32 * NS;
  constexpr int ARow = 2 * kBlock;    // bf16 C bytes per row per K block
  constexpr int AI = BM / 4;          // C DMA instructions per step (4 rows x 256 B each)
  constexpr int BI = BN / 8;          // W2 DMA instructions per step (8 rows x 128 B each)
  constexpr int OPS = AI + BI;
  constexpr int MW = MS + 2;          // compute-wave metadata dwords per lane
  constexpr int ASZ = BM * ARow, BSZ = BN * kBlock;
  __shared__ __attribute__((aligned(16))) uint8_t aring[D][ASZ];
  __shared__ __attribute__((aligned(16))) uint8_t bring[D][BSZ];
  __shared__ __attribute__((aligned(16))) float mring[kComputeWaves][MW][kWave];

  const int lane = threadIdx.x & (kWave - 1), w = wave_id();
  const int NNT = H / BN, NKB = I / kBlock;
  TileMap tm;
  tm.init(counts, offsets, E_l, BM);
  const int items = tm.total * NNT;
  int it = uniform((int)blockIdx.x);
  if (it >= items) return;
  const int stride = gridDim.x;

  auto scalars = [&](int item, B2Scalars& x) {
    item = uniform(item);
    const int tile = item / NNT, nt = item % NNT;
    x.e = uniform(tm.find(tile, BM, x.m0, x.cnt, x.seg));
    x.m0 = uniform(x.m0);
    x.cnt = uniform(x.cnt);
    x.seg = uniform(x.seg);
    x.h0 = uniform((uint32_t)(nt * BN));
    x.wbase = uniform(w2 + (size_t)x.e * H * I);
  };
  int it_n = it + stride;

  if (w == kProducer) {
    const __amdgpu_buffer_rsrc_t cres = make_rsrc(C, (uint32_t)max_pairs * I * 2);
    const uint32_t dma0 = wblk_dma_off(lane, 0, I), dma1 = wblk_dma_off(lane, 1, I);
    struct P {
      B2Scalars s;
      uint32_t aoff[AI];
    };
    // C DMA instruction j covers tile rows 4j + lane/16, chunk position lane & 15 holding
    // chunk (lane & 15) ^ (row & 15).
    auto meta = [&](int item, P& x) {
      scalars(item, x.s);
      const int last = x.s.cnt - 1;
#pragma unroll
      for (int j = 0; j < AI; ++j) {
        const int row = 4 * j + (lane >> 4);
        const int r = x.s.m0 + row;
        x.aoff[j] = ((uint32_t)(x.s.seg + (r < last ? r : last)) * I) * 2 +
                    16 * ((lane & 15) ^ (row & 15));
      }
    };
    P cur, nxt, nn;
    meta(it, cur);
    meta(it_n < items ? it_n : it, nxt);
    auto issue = [&](bool second, int kbi, int slot) {
      const P& x = second ? nxt : cur;
#pragma unroll
      for (int j = 0; j < AI; ++j)
        dma16(cres, &aring[slot][j * 1024], second ? nxt.aoff[j] : cur.aoff[j],
              (uint32_t)kbi * ARow);
      const __amdgpu_buffer_rsrc_t wres = make_rsrc(uniform(x.s.wbase), (uint32_t)H * I);
      const uint32_t h0 = uniform(x.s.h0);
#pragma unroll
      for (int j = 0; j < BI; ++j)
        dma16(wres, &bring[slot][j * 1024], (j & 1) ? dma1 : dma0,
              uniform((h0 + 16 * (j >> 1)) * (uint32_t)I + (uint32_t)kbi * kBlock));
    };
#pragma unroll
    for (int d = 0; d < D - 1; ++d) {
      issue(false, d, d);
      __builtin_amdgcn_sched_barrier(0);
    }
    int slot = 0;
    for (;;) {
      const int it_nn = it_n + stride;
      meta(it_nn < items ? it_nn : (it_n < items ? it_n : it), nn);
      int kb = 0;
      do {
        vm_wait<vm_depth((D - 2) * OPS)>();
        __builtin_amdgcn_s_barrier();
        const int kn = kb + D - 1;
        const bool second = kn >= NKB;
        issue(second, second ? kn - NKB : kn, slot == 0 ? D - 1 : slot - 1);
        __builtin_amdgcn_sched_barrier(0);
        slot = slot + 1 == D ? 0 : slot + 1;
        ++kb;
      } while (kb < NKB);
      if (it_n >= items) break;
      it = it_n;
      it_n = it_nn;
      cur = nxt;
      nxt = nn;
    }
    vm_wait<0>();
    return;
  }

  const int wm = w & 1, wn = w >> 1;
  const int r16 = lane & 15, g = lane >> 4;
  const __amdgpu_buffer_rsrc_t wgtres = make_rsrc(sorted_w, (uint32_t)max_pairs * 4);
  const __amdgpu_buffer_rsrc_t s2res = make_rsrc(s2, (uint32_t)E_l * (H / kBlock) * NKB * 4);
  const uint32_t rd0 = wblk_read_off(lane, 0), rd1 = wblk_read_off(lane, 1);
  float* my_meta = &mring[w][0][0];
  struct Q {
    B2Scalars s;
    LaneScales sc;  // weight scales of this wave's columns (one 128-block)
    float wgt[MS];  // routing weight of the lane's output row in each sub-tile
  };
  auto meta = [&](int item, Q& x) {
    scalars(item, x.s);
    const int last = x.s.cnt - 1;
#pragma unroll
    for (int ms = 0; ms < MS; ++ms) {
      const int r = x.s.m0 + (wm * MS + ms) * 16 + r16;
      dma4(wgtres, my_meta + ms * kWave, 4u * (x.s.seg + (r < last ? r : last)), 0);
    }
    const int wc = x.s.h0 + wn * 16 * NS;
    const uint32_t so =
        uniform((uint32_t)(((size_t)x.s.e * (H / kBlock) + wc / kBlock) * NKB) * 4);
    dma4(s2res, my_meta + MS * kWave, 4u * lane, so);
    dma4(s2res, my_meta + (MS + 1) * kWave, 4u * (lane + kWave), so);
  };
  auto finish = [&](Q& x) {
    const uint32_t mb = lds_addr(my_meta) + 4 * lane;
    float v[MW];
#pragma unroll
    for (int j = 0; j < MW; ++j) v[j] = ds_read4f(mb + j * 4 * kWave);
    lds_wait_all();
#pragma unroll
    for (int j = 0; j < MW; ++j) lds_fence(v[j]);
#pragma unroll
    for (int ms = 0; ms < MS; ++ms) x.wgt[ms] = v[ms];
    x.sc.v0 = v[MS];
    x.sc.v1 = v[MS + 1];
  };
  Q cur, nxt, nn;
  meta(it, cur);
  vm_wait<0>();
  finish(cur);
  meta(it_n < items ? it_n : it, nxt);
  vm_wait<0>();
  finish(nxt);

  int slot = 0;
  for (;;) {
    const int it_nn = it_n + stride;
    meta(it_nn < items ? it_nn : (it_n < items ? it_n : it), nn);
    v4f acc[MS][NS];
#pragma unroll
    for (int ms = 0; ms < MS; ++ms)
#pragma unroll
      for (int ns = 0; ns < NS; ++ns) acc[ms][ns] = v4f{0.f, 0.f, 0.f, 0.f};
    int kb = 0;
    do {
      const int d = slot;
      __builtin_amdgcn_s_barrier();
      const uint32_t ab = lds_addr(&aring[d][0]);
      const uint32_t bb = lds_addr(&bring[d][0]) + wn * NS * kWBlk;
      v4u wl[NS], wh[NS];
#pragma unroll
      for (int ns = 0; ns < NS; ++ns) {
        wl[ns] = ds_read16(bb + ns * kWBlk + rd0);
        wh[ns] = ds_read16(bb + ns * kWBlk + rd1);
      }
      auto read_a = [&](int ms, v4u (&a)[4]) {
        const int row = (wm * MS + ms) * 16 + r16;
#pragma unroll
        for (int c = 0; c < 4; ++c)
          a[c] = ds_read16(ab + row * ARow + 16 * ((4 * g + c) ^ (row & 15)));
      };
      v4u a[4];
      read_a(0, a);
      const float sw = cur.sc.get(kb);
      lds_wait_all();
      v8bf bw[NS][4];
#pragma unroll
      for (int ns = 0; ns < NS; ++ns) {
        lds_fence(wl[ns]);
        lds_fence(wh[ns]);
        const uint32_t wv[8] = {wl[ns][0], wl[ns][1], wl[ns][2], wl[ns][3],
                                wh[ns][0], wh[ns][1], wh[ns][2], wh[ns][3]};
#pragma unroll
        for (int c = 0; c < 4; ++c) {
          v2bf p0, p1, p2, p3;
          fp8x4_to_bf16x4((int)wv[2 * c], p0, p1);
          fp8x4_to_bf16x4((int)wv[2 * c + 1], p2, p3);
          bw[ns][c] = v8bf{p0[0], p0[1], p1[0], p1[1], p2[0], p2[1], p3[0], p3[1]};
        }
      }
#pragma unroll
      for (int c = 0; c < 4; ++c) lds_fence(a[c]);
#pragma unroll
      for (int ms = 0; ms < MS; ++ms) {
        v8bf av[4];
#pragma unroll
        for (int c = 0; c < 4; ++c) av[c] = __builtin_bit_cast(v8bf, a[c]);
        if (ms + 1 < MS) read_a(ms + 1, a);
#pragma unroll
        for (int ns = 0; ns < NS; ++ns) {
          v4f t = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
          for (int c = 0; c < 4; ++c) t = mfma_bf16_16x16x32(bw[ns][c], av[c], t);
#pragma unroll
          for (int i = 0; i < 4; ++i) acc[ms][ns][i] = fmaf(t[i], sw, acc[ms][ns][i]);
        }
        if (ms + 1 < MS) {
          lds_wait_all();
#pragma unroll
          for (int c = 0; c < 4; ++c) lds_fence(a[c]);
        }
      }
      slot = slot + 1 == D ? 0 : slot + 1;
      ++kb;
    } while (kb < NKB);
    vm_wait<0>();
    finish(nn);

#pragma unroll
    for (int ms = 0; ms < MS; ++ms) {
      const int r = cur.s.m0 + (wm * MS + ms) * 16 + r16;
      if (r < cur.s.cnt) {
        const float wp = cur.wgt[ms];
        float* orow = partial + (size_t)(cur.s.seg + r) * H + cur.s.h0 + wn * 16 * NS + 4 * g;
#pragma unroll
        for (int ns = 0; ns < NS; ++ns)
          *(float4*)(orow + 16 * ns) = float4{acc[ms][ns][0] * wp, acc[ms][ns][1] * wp,
                                              acc[ms][ns][2] * wp, acc[ms][ns][3] * wp};
      }
    }
    if (it_n >= items) break;
    it = it_n;
    it_n = it_nn;
    cur = nxt;
    nxt = nn;
  }
}

}  // namespace

static int big_grid(long long max_items) {
  static int cus = 0;
  if (cus == 0) {
    int dev = 0, n = 0;
    cus = (hipGetDevice(&dev) == hipSuccess &&
           hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) == hipSuccess &&
           n > 0)
              ? n
              : 256;
  }
  long long g = cus;  // the LDS rings leave room for one workgroup per CU
  if (g > max_items) g = max_items;
  return g < 1 ? 1 : (int)g;
}

static inline long long big_tiles(int max_pairs, int bm, int E_l) {
  return (max_pairs + bm - 1) / bm + (E_l < max_pairs ? E_l : max_pairs);
}

#ifndef JG_B1_MS
#define JG_B1_MS 4
#endif
#ifndef JG_B1_NS
#define JG_B1_NS 4
#endif
#ifndef JG_B1_D
#define JG_B1_D 3
#endif
#ifndef JG_B2_MS
#define JG_B2_MS 4
#endif
#ifndef JG_B2_NS
#define JG_B2_NS 4
#endif
#ifndef JG_B2_D
#define JG_B2_D 3
#endif

hipError_t launch_gemm1_big(const uint8_t* hs, const float* hs_scale, const uint8_t* w13,
                            const float* s13, const int32_t* counts, const int32_t* offsets,
                            const int32_t* sorted_tok, uint16_t* C, int T, int H, int I, int E_l,
                            int max_pairs, hipStream_t stream) {
  constexpr int BN = 32 * JG_B1_NS;
  if (I % BN != 0 || H / kBlock < JG_B1_D - 1) return hipErrorNotSupported;
  const int grid = big_grid(big_tiles(max_pairs, 32 * JG_B1_MS, E_l) * (I / BN));
  gemm1_big_kernel<JG_B1_MS, JG_B1_NS, JG_B1_D><<<grid, (kComputeWaves + 1) * kWave, 0, stream>>>(
      hs, hs_scale, w13, s13, counts, offsets, sorted_tok, C, T, H, I, E_l, max_pairs);
  return hipGetLastError();
}

hipError_t launch_gemm2_big(const uint16_t* C, const uint8_t* w2, const float* s2,
                            const int32_t* counts, const int32_t* offsets, const float* sorted_w,
                            float* partial, int H, int I, int E_l, int max_pairs,
                            hipStream_t stream) {
  constexpr int BN = 32 * JG_B2_NS;
  if (H % BN != 0 || I / kBlock < JG_B2_D - 1) return hipErrorNotSupported;
  const int grid = big_grid(big_tiles(max_pairs, 32 * JG_B2_MS, E_l) * (H / BN));
  gemm2_big_kernel<JG_B2_MS, JG_B2_NS, JG_B2_D><<<grid, (kComputeWaves + 1) * kWave, 0, stream>>>(
      C, w2, s2, counts, offsets, sorted_w, partial, H, I, E_l, max_pairs);
  return hipGetLastError();
}

}  // namespace jgmoe
