// LDS-tiled grouped GEMM1 + SwiGLU for segments of 2..15 expected pairs per expert (32-row
// tiles; from 16 the large-tile kernel's 64-row tiles are faster), and the LDS-tiled GEMM2 for
// segments of up to 7.
//
// A workgroup (4 waves) computes a BM x 64 tile of one expert's GEMM1 output (BM = 16*MT pairs).
// Everything reaches LDS by DMA (buffer_load ... lds), so the only VGPRs spent on memory are the
// MFMA fragments of the current K block:
//
// * The activation tile (BM fp8 hidden-state rows x one 128-wide K block) is gathered straight
//   from the token rows into a ring of D LDS slots shared by the four waves, each wave issuing a
//   quarter of the DMA instructions, with the rows' activation scales (4-byte DMA).
// * Each wave streams the weight rows of its own 16 output columns (X1 and X2) into a private
//   ring.
// * One barrier per K step: a wave waits for its own DMAs of the step's block (counted vmcnt),
//   the barrier makes everyone's visible and frees the slot read in the previous step, which is
//   refilled at once with the block D-1 steps ahead. The prefetch runs across item boundaries
//   (the wave's next item is resolved one item ahead), so the stream never drains.
//
// LDS images are XOR-swizzled in 16-byte chunks (the DMA lane -> global address map does the
// permutation) so MFMA fragment reads are bank-conflict free. MFMA forms, scale handling and
// epilogues are those of the stream kernels.
#include "moe_device.h"
#include "moe_kernels.h"

namespace jgmoe {

namespace {

constexpr int kWaves = 4;
constexpr int kWBlk = 16 * kBlock;  // 16 weight rows x 128 bytes

// vmcnt holds 6 bits; deeper counts are clamped, which only makes a wait stricter.
constexpr int vm_depth(int n) { return n > 63 ? 63 : n < 0 ? 0 : n; }

// ---- GEMM1 ------------------------------------------------------------------------------------

template <int MT>
struct T1Item {
  const uint8_t* wbase;   // the expert's W13
  uint32_t wsoff;         // c0 * H (this wave's first X1 row)
  LaneScales sc1, sc2;    // weight scales of this wave's X1 / X2 row block
  uint32_t aoff[MT / 2];  // per lane: global offset of its A DMA chunk (token row, K 0)
  uint32_t saoff;         // per lane: token * 4 for its activation-scale DMA
  int m0, cnt, seg, c0;
};

template <int MT, int D>
__global__ __launch_bounds__(256) void gemm1_tile_kernel(
    const uint8_t* __restrict__ hs, const float* __restrict__ hs_scale,
    const uint8_t* __restrict__ w13, const float* __restrict__ s13,
    const int32_t* __restrict__ counts, const int32_t* __restrict__ offsets,
    const int32_t* __restrict__ sorted_tok, uint16_t* __restrict__ C, int T, int H, int I,
    int E_l, int max_pairs) {
  static_assert(MT % 2 == 0 && MT <= 8, "A DMA splits BM rows over 4 waves, 8 rows each");
  static_assert(D >= 3, "the prefetch lead is D-1 blocks");
  constexpr int BM = 16 * MT;
  constexpr int AI = MT / 2;        // A DMA instructions per wave per step (8 rows x 128 B each)
  constexpr int OPS = 4 + AI + 1;   // vector-memory operations per wave per step
  constexpr int MW = AI + 5;        // metadata dwords per lane
  __shared__ __attribute__((aligned(16))) uint32_t mring[kWaves][MW][kWave];
  __shared__ __attribute__((aligned(16))) uint8_t bring[kWaves][D][2 * kWBlk];
  __shared__ __attribute__((aligned(16))) uint8_t aring[D][BM * kBlock];
  // Each wave's scale DMA writes 64 dwords (one per lane) from row (w*64) mod BM, so a slot
  // holds at least 64 floats even when BM = 32 (lanes past the tile repeat its last row).
  constexpr int SROW = BM < kWave ? kWave : BM;
  __shared__ __attribute__((aligned(16))) float sring[D][SROW];

  const int lane = threadIdx.x & (kWave - 1), w = wave_id();
  const int r16 = lane & 15, g = lane >> 4;
  const int NNT = I / 64, NKB = H / kBlock;
  TileMap tm;
  tm.init(counts, offsets, E_l, BM);
  const int items = tm.total * NNT;
  int it = uniform((int)blockIdx.x);
  if (it >= items) return;  // whole workgroup
  const int stride = gridDim.x;

  const __amdgpu_buffer_rsrc_t ares = make_rsrc(hs, (uint32_t)T * H);
  const __amdgpu_buffer_rsrc_t sares = make_rsrc(hs_scale, (uint32_t)T * NKB * 4);
  const uint32_t dma0 = wblk_dma_off(lane, 0, H), dma1 = wblk_dma_off(lane, 1, H);
  const uint32_t rd0 = wblk_read_off(lane, 0), rd1 = wblk_read_off(lane, 1);
  uint8_t* my_bring = &bring[w][0][0];

  // Per-lane item metadata (token ids of the rows this wave's DMAs fetch, weight-scale rows)
  // arrives by 4-byte DMA in a small per-wave LDS area and is read back at the item switch, so
  // the compiler tracks no loads across the K loop. A instruction i covers tile rows
  // 8*(w*AI + i) + lane/8; the scale DMA covers row (w*64) mod BM + lane (clamped to the tile).
  const __amdgpu_buffer_rsrc_t tokres = make_rsrc(sorted_tok, (uint32_t)max_pairs * 4);
  const __amdgpu_buffer_rsrc_t s13res =
      make_rsrc(s13, (uint32_t)E_l * (2 * I / kBlock) * NKB * 4);
  uint32_t* my_meta = &mring[w][0][0];
  auto meta = [&](int item, T1Item<MT>& x) {
    item = uniform(item);
    const int tile = item / NNT, nt = item % NNT;
    const int e = tm.find(tile, BM, x.m0, x.cnt, x.seg);
    x.m0 = uniform(x.m0);
    x.cnt = uniform(x.cnt);
    x.seg = uniform(x.seg);
    x.c0 = uniform(nt * 64 + w * 16);
    x.wbase = uniform(w13 + (size_t)e * 2 * I * H);
    x.wsoff = uniform((uint32_t)x.c0 * H);
    const int last = x.cnt - 1;
#pragma unroll
    for (int i = 0; i < AI; ++i) {
      const int r = x.m0 + 8 * (w * AI + i) + (lane >> 3);
      dma4(tokres, my_meta + i * kWave, 4u * (x.seg + (r < last ? r : last)), 0);
    }
    // Waves whose 64 rows lie past BM repeat the rows of wave w mod (BM/64): same bytes to the
    // same LDS words, so every wave issues the same operation count.
    const int rs = x.m0 + (w * kWave) % BM + (lane < BM ? lane : BM - 1);
    dma4(tokres, my_meta + AI * kWave, 4u * (x.seg + (rs < last ? rs : last)), 0);
    const uint32_t so1 = uniform((uint32_t)((e * (2 * I / kBlock) + x.c0 / kBlock) * NKB) * 4);
    const uint32_t so2 =
        uniform((uint32_t)((e * (2 * I / kBlock) + (I + x.c0) / kBlock) * NKB) * 4);
    dma4(s13res, my_meta + (AI + 1) * kWave, 4u * lane, so1);
    dma4(s13res, my_meta + (AI + 2) * kWave, 4u * (lane + kWave), so1);
    dma4(s13res, my_meta + (AI + 3) * kWave, 4u * lane, so2);
    dma4(s13res, my_meta + (AI + 4) * kWave, 4u * (lane + kWave), so2);
  };
  // Reads back the per-lane metadata of the last meta() (its DMAs must have completed).
  auto finish = [&](T1Item<MT>& x) {
    const uint32_t mb = lds_addr(my_meta) + 4 * lane;
    float v[MW];
#pragma unroll
    for (int j = 0; j < MW; ++j) v[j] = ds_read4f(mb + j * 4 * kWave);
    lds_wait_all();
#pragma unroll
    for (int j = 0; j < MW; ++j) lds_fence(v[j]);
#pragma unroll
    for (int i = 0; i < AI; ++i) {
      const int row = 8 * (w * AI + i) + (lane >> 3);
      x.aoff[i] = __float_as_uint(v[i]) * H + 16 * ((lane & 7) ^ wblk_swz(row));
    }
    x.saoff = __float_as_uint(v[AI]) * 4;
    x.sc1.v0 = v[AI + 1];
    x.sc1.v1 = v[AI + 2];
    x.sc2.v0 = v[AI + 3];
    x.sc2.v1 = v[AI + 4];
  };

  T1Item<MT> cur, nxt, nn;
  meta(it, cur);
  vm_wait<0>();
  finish(cur);
  int it_n = it + stride;
  meta(it_n < items ? it_n : it, nxt);
  vm_wait<0>();
  finish(nxt);

  auto issue = [&](bool second, int kbi, int slot) {
#pragma unroll
    for (int i = 0; i < AI; ++i)
      dma16(ares, &aring[slot][(w * AI + i) * 1024], second ? nxt.aoff[i] : cur.aoff[i],
            (uint32_t)kbi * kBlock);
    dma4(sares, &sring[slot][(w * kWave) % BM], second ? nxt.saoff : cur.saoff,
         (uint32_t)kbi * T * 4);
    const __amdgpu_buffer_rsrc_t wres =
        make_rsrc(uniform(second ? nxt.wbase : cur.wbase), 2u * I * H);
    const uint32_t ws = uniform((second ? nxt.wsoff : cur.wsoff) + (uint32_t)kbi * kBlock);
    uint8_t* b = my_bring + slot * 2 * kWBlk;
    dma16_stream(wres, b, dma0, ws);
    dma16_stream(wres, b + 1024, dma1, ws);
    dma16_stream(wres, b + kWBlk, dma0, ws + (uint32_t)I * H);
    dma16_stream(wres, b + kWBlk + 1024, dma1, ws + (uint32_t)I * H);
  };

  // Blocks 0..D-2 of the first item; block s+D-1 is issued at step s.
#pragma unroll
  for (int d = 0; d < D - 1; ++d) {
    issue(false, d, d);
    __builtin_amdgcn_sched_barrier(0);
  }

  int slot = 0;  // ring slot of the next block to compute (a running step count mod D)
  for (;;) {
    const int it_nn = it_n + stride;
    meta(it_nn < items ? it_nn : (it_n < items ? it_n : it), nn);

    v4f acc1[MT], acc2[MT];
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
      acc1[mt] = v4f{0.f, 0.f, 0.f, 0.f};
      acc2[mt] = v4f{0.f, 0.f, 0.f, 0.f};
    }
    int kb = 0;
    do {
      {
        const int d = slot;
        vm_wait<vm_depth((D - 2) * OPS)>();  // this wave's DMAs of block kb are done
        // Everyone's are, and everyone has finished reading slot d-1. A bare s_barrier: the
        // fence of __syncthreads would wait for every DMA in flight.
        __builtin_amdgcn_s_barrier();
        const int kn = kb + D - 1;
        const bool second = kn >= NKB;
        issue(second, second ? kn - NKB : kn, d == 0 ? D - 1 : d - 1);
        __builtin_amdgcn_sched_barrier(0);

        const uint32_t bb = lds_addr(my_bring + d * 2 * kWBlk);
        const uint32_t ab = lds_addr(&aring[d][0]);
        const uint32_t sb = lds_addr(&sring[d][0]);
        v4u x1l = ds_read16(bb + rd0), x1h = ds_read16(bb + rd1);
        v4u x2l = ds_read16(bb + kWBlk + rd0), x2h = ds_read16(bb + kWBlk + rd1);
        v4u al[MT], ah[MT];
        float sa[MT];
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) {
          al[mt] = ds_read16(ab + mt * kWBlk + rd0);
          ah[mt] = ds_read16(ab + mt * kWBlk + rd1);
          sa[mt] = ds_read4f(sb + 4 * (mt * 16 + r16));
        }
        lds_wait_all();
        lds_fence(x1l);
        lds_fence(x1h);
        lds_fence(x2l);
        lds_fence(x2h);
        const v8i b1 = v8i{(int)x1l[0], (int)x1l[1], (int)x1l[2], (int)x1l[3],
                           (int)x1h[0], (int)x1h[1], (int)x1h[2], (int)x1h[3]};
        const v8i b2 = v8i{(int)x2l[0], (int)x2l[1], (int)x2l[2], (int)x2l[3],
                           (int)x2h[0], (int)x2h[1], (int)x2h[2], (int)x2h[3]};
        const float sw1 = cur.sc1.get(kb), sw2 = cur.sc2.get(kb);
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) {
          lds_fence(al[mt]);
          lds_fence(ah[mt]);
          lds_fence(sa[mt]);
          const v8i a = v8i{(int)al[mt][0], (int)al[mt][1], (int)al[mt][2], (int)al[mt][3],
                            (int)ah[mt][0], (int)ah[mt][1], (int)ah[mt][2], (int)ah[mt][3]};
          const float f1 = sa[mt] * sw1, f2 = sa[mt] * sw2;
          const v4f p = mfma_f8_16x16x128(b1, a);
          const v4f q = mfma_f8_16x16x128(b2, a);
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            acc1[mt][i] = fmaf(p[i], f1, acc1[mt][i]);
            acc2[mt][i] = fmaf(q[i], f2, acc2[mt][i]);
          }
        }
      }
      slot = slot + 1 == D ? 0 : slot + 1;
      ++kb;
    } while (kb < NKB);
    // Everything but the next item's prefetched blocks is complete, the metadata DMAs included.
    vm_wait<vm_depth((D - 1) * OPS)>();
    finish(nn);

#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
      const int r = cur.m0 + mt * 16 + r16;
      if (r < cur.cnt) {
        uint32_t h[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const float x1 = acc1[mt][i], x2 = acc2[mt][i];
          h[i] = float_to_bf16_bits(x1 * (x2 / (1.0f + __expf(-x2))));
        }
        *(uint2*)(C + (size_t)(cur.seg + r) * I + cur.c0 + 4 * g) =
            uint2{h[0] | (h[1] << 16), h[2] | (h[3] << 16)};
      }
    }
    if (it_n >= items) break;
    it = it_n;
    it_n = it_nn;
    cur = nxt;
    nxt = nn;
  }
  vm_wait<0>();  // no DMA may still target this workgroup's LDS when it retires
}


// ---- GEMM2 ------------------------------------------------------------------------------------
//
// A workgroup (4 waves) computes a BM x 64 tile of one expert's GEMM2 output (BM = 16*MT pairs):
// the BM bf16 C rows of a K block are shared by the four waves through one LDS ring (each wave
// DMAs a quarter of them; the tile's buffer resource ends at the segment, so padding rows are
// never fetched), each wave streams the W2 rows of its own 16 output columns into a private ring
// (non-temporal: read once per call). Same per-step barrier protocol as GEMM1 above; MFMA form,
// scales and epilogue as in the streaming GEMM2.

template <int MT>
struct T2Item {
  const uint8_t* wbase;   // the expert's W2
  uint32_t wsoff;         // h0 * I (this wave's first W2 row)
  LaneScales sc;          // weight scales of this wave's 128-row W2 block
  float wgt[MT];          // routing weight of the lane's row in each sub-tile
  int dst[MT];            // destination row code (pair_dst) of that row
  const uint16_t* cbase;  // C row of the tile's first pair
  uint32_t crec;          // bytes of C from cbase to the segment's end
  int m0, cnt, seg, h0;
};

template <int MT, int D>
__global__ __launch_bounds__(256) void gemm2_tile_kernel(
    const uint16_t* __restrict__ C, const uint8_t* __restrict__ w2, const float* __restrict__ s2,
    const int32_t* __restrict__ counts, const int32_t* __restrict__ offsets,
    const float* __restrict__ sorted_w, Gemm2Out dst, int H, int I, int E_l, int max_pairs) {
  static_assert(D >= 3, "the prefetch lead is D-1 blocks");
  constexpr int BM = 16 * MT;
  constexpr int ARow = 2 * kBlock;  // bf16 C bytes per row per K block
  constexpr int AI = MT;            // C DMA instructions per wave per step (4 rows x 256 B each)
  constexpr int OPS = AI + 2;       // vector-memory operations per wave per step
  constexpr int MW = 2 * MT + 2;    // metadata dwords per lane
  __shared__ __attribute__((aligned(16))) uint32_t mring[kWaves][MW][kWave];
  __shared__ __attribute__((aligned(16))) uint8_t bring[kWaves][D][kWBlk];
  __shared__ __attribute__((aligned(16))) uint8_t aring[D][BM * ARow];

  const int lane = threadIdx.x & (kWave - 1), w = wave_id();
  const int r16 = lane & 15, g = lane >> 4;
  const int NNT = H / 64, NKB = I / kBlock;
  TileMap tm;
  tm.init(counts, offsets, E_l, BM);
  const int items = tm.total * NNT;
  int it = uniform((int)blockIdx.x);
  if (it >= items) return;  // whole workgroup
  const int stride = gridDim.x;

  const uint32_t dma0 = wblk_dma_off(lane, 0, I), dma1 = wblk_dma_off(lane, 1, I);
  const uint32_t rd0 = wblk_read_off(lane, 0), rd1 = wblk_read_off(lane, 1);
  uint8_t* my_bring = &bring[w][0][0];
  // C DMA instruction i of wave w covers tile rows 4*(w*AI + i) + lane/16, chunk position
  // lane & 15 holding chunk (lane & 15) ^ crow_swz(row); offsets relative to the tile's first row.
  uint32_t aoff[AI];
#pragma unroll
  for (int i = 0; i < AI; ++i) {
    const int row = 4 * (w * AI + i) + (lane >> 4);
    aoff[i] = (uint32_t)row * I * 2 + 16 * ((lane & 15) ^ crow_swz(row));
  }

  const __amdgpu_buffer_rsrc_t wgtres = make_rsrc(sorted_w, (uint32_t)max_pairs * 4);
  const __amdgpu_buffer_rsrc_t dstres = make_rsrc(dst.pair_dst, (uint32_t)max_pairs * 4);
  const __amdgpu_buffer_rsrc_t s2res = make_rsrc(s2, (uint32_t)E_l * (H / kBlock) * NKB * 4);
  uint32_t* my_meta = &mring[w][0][0];
  auto meta = [&](int item, T2Item<MT>& x) {
    item = uniform(item);
    const int tile = item / NNT, nt = item % NNT;
    const int e = tm.find(tile, BM, x.m0, x.cnt, x.seg);
    x.m0 = uniform(x.m0);
    x.cnt = uniform(x.cnt);
    x.seg = uniform(x.seg);
    x.h0 = uniform(nt * 64 + w * 16);
    x.wbase = uniform(w2 + (size_t)e * H * I);
    x.wsoff = uniform((uint32_t)x.h0 * I);
    x.cbase = uniform(C + (size_t)(x.seg + x.m0) * I);
    x.crec = uniform((uint32_t)(x.cnt - x.m0) * I * 2);
    const int last = x.cnt - 1;
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
      const int r = x.m0 + mt * 16 + r16;
      const uint32_t p = 4u * (x.seg + (r < last ? r : last));
      dma4(wgtres, my_meta + mt * kWave, p, 0);
      dma4(dstres, my_meta + (MT + mt) * kWave, p, 0);
    }
    const uint32_t so = uniform((uint32_t)((e * (H / kBlock) + x.h0 / kBlock) * NKB) * 4);
    dma4(s2res, my_meta + 2 * MT * kWave, 4u * lane, so);
    dma4(s2res, my_meta + (2 * MT + 1) * kWave, 4u * (lane + kWave), so);
  };
  auto finish = [&](T2Item<MT>& x) {
    const uint32_t mb = lds_addr(my_meta) + 4 * lane;
    float v[MW];
#pragma unroll
    for (int j = 0; j < MW; ++j) v[j] = ds_read4f(mb + j * 4 * kWave);
    lds_wait_all();
#pragma unroll
    for (int j = 0; j < MW; ++j) lds_fence(v[j]);
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
      x.wgt[mt] = v[mt];
      x.dst[mt] = __float_as_int(v[MT + mt]);
    }
    x.sc.v0 = v[2 * MT];
    x.sc.v1 = v[2 * MT + 1];
  };

  T2Item<MT> cur, nxt, nn;
  int it_n = it + stride;
  auto issue = [&](bool second, int kbi, int slot) {
    const __amdgpu_buffer_rsrc_t cres = make_rsrc(uniform(second ? nxt.cbase : cur.cbase),
                                                  uniform(second ? nxt.crec : cur.crec));
#pragma unroll
    for (int i = 0; i < AI; ++i)
      dma16(cres, &aring[slot][(w * AI + i) * 1024], aoff[i], (uint32_t)kbi * ARow);
    const __amdgpu_buffer_rsrc_t wres =
        make_rsrc(uniform(second ? nxt.wbase : cur.wbase), (uint32_t)H * I);
    const uint32_t ws = uniform((second ? nxt.wsoff : cur.wsoff) + (uint32_t)kbi * kBlock);
    uint8_t* b = my_bring + slot * kWBlk;
    dma16_stream(wres, b, dma0, ws);
    dma16_stream(wres, b + 1024, dma1, ws);
  };

  // The prologue's DMAs need only the tile map, so they go out with the first item's metadata
  // DMAs instead of after them: the weight stream starts one round trip sooner (DS-V3 T=16 call
  // 62.6 -> 62.1 us; T=64 unchanged).
  meta(it, cur);
#pragma unroll
  for (int d = 0; d < D - 1; ++d) {
    issue(false, d, d);
    __builtin_amdgcn_sched_barrier(0);
  }
  vm_wait<vm_depth((D - 1) * OPS)>();  // the metadata DMAs, issued first, have landed
  finish(cur);
  meta(it_n < items ? it_n : it, nxt);
  vm_wait<0>();
  finish(nxt);

  int slot = 0;
  for (;;) {
    const int it_nn = it_n + stride;
    meta(it_nn < items ? it_nn : (it_n < items ? it_n : it), nn);

    v4f acc[MT];
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) acc[mt] = v4f{0.f, 0.f, 0.f, 0.f};
    int kb = 0;
    do {
      {
        const int d = slot;
        vm_wait<vm_depth((D - 2) * OPS)>();  // this wave's DMAs of block kb are done
        __builtin_amdgcn_s_barrier();        // everyone's are; slot d-1 is no longer read
        const int kn = kb + D - 1;
        const bool second = kn >= NKB;
        issue(second, second ? kn - NKB : kn, d == 0 ? D - 1 : d - 1);
        __builtin_amdgcn_sched_barrier(0);

        const uint32_t bb = lds_addr(my_bring + d * kWBlk);
        const uint32_t ab = lds_addr(&aring[d][0]);
        v4u wl = ds_read16(bb + rd0), wh = ds_read16(bb + rd1);
        v4u a[MT][4];
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) {
          const int row = mt * 16 + r16;
#pragma unroll
          for (int c = 0; c < 4; ++c)
            a[mt][c] = ds_read16(ab + row * ARow + 16 * ((4 * g + c) ^ crow_swz(row)));
        }
        lds_wait_all();
        lds_fence(wl);
        lds_fence(wh);
        const uint32_t wv[8] = {wl[0], wl[1], wl[2], wl[3], wh[0], wh[1], wh[2], wh[3]};
        v8bf bw[4];
#pragma unroll
        for (int c = 0; c < 4; ++c) {
          v2bf p0, p1, p2, p3;
          fp8x4_to_bf16x4((int)wv[2 * c], p0, p1);
          fp8x4_to_bf16x4((int)wv[2 * c + 1], p2, p3);
          bw[c] = v8bf{p0[0], p0[1], p1[0], p1[1], p2[0], p2[1], p3[0], p3[1]};
        }
        const float sw = cur.sc.get(kb);
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) {
          v4f t = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
          for (int c = 0; c < 4; ++c) {
            lds_fence(a[mt][c]);
            t = mfma_bf16_16x16x32(bw[c], __builtin_bit_cast(v8bf, a[mt][c]), t);
          }
#pragma unroll
          for (int i = 0; i < 4; ++i) acc[mt][i] = fmaf(t[i], sw, acc[mt][i]);
        }
      }
      slot = slot + 1 == D ? 0 : slot + 1;
      ++kb;
    } while (kb < NKB);
    vm_wait<vm_depth((D - 1) * OPS)>();  // the next item's metadata DMAs have landed
    finish(nn);

#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
      const int r = cur.m0 + mt * 16 + r16;
      if (r < cur.cnt) {
        const float wp = cur.wgt[mt];
        const int dd = cur.dst[mt];
        uint16_t* row = dd >= 0 ? dst.out + (size_t)dd * H : dst.partial + (size_t)(-1 - dd) * H;
        const uint32_t h01 = (uint32_t)float_to_bf16_bits(acc[mt][0] * wp) |
                             ((uint32_t)float_to_bf16_bits(acc[mt][1] * wp) << 16);
        const uint32_t h23 = (uint32_t)float_to_bf16_bits(acc[mt][2] * wp) |
                             ((uint32_t)float_to_bf16_bits(acc[mt][3] * wp) << 16);
        *(uint2*)(row + cur.h0 + 4 * g) = uint2{h01, h23};
      }
    }
    if (it_n >= items) break;
    it = it_n;
    it_n = it_nn;
    cur = nxt;
    nxt = nn;
  }
  vm_wait<0>();  // no DMA may still target this workgroup's LDS when it retires
}

}  // namespace

static int tile_grid(int per_cu, long long max_items) {
  const int cus = device_cu_count();
  long long g = (long long)cus * per_cu;
  if (g > max_items) g = max_items;
  return g < 1 ? 1 : (int)g;
}

// Workgroups per CU that fit the LDS rings (160 KiB per CU).
static inline int tile_groups_per_cu(int lds_bytes) {
  const int n = (160 * 1024) / lds_bytes;
  return n < 1 ? 1 : n > 4 ? 4 : n;
}

static inline long long tile_count(int max_pairs, int bm, int E_l) {
  return (max_pairs + bm - 1) / bm + (E_l < max_pairs ? E_l : max_pairs);
}

// Ring depths (lead D-1 blocks). D = 3 keeps two workgroups per CU within the 160 KiB of LDS,
// which measured faster than deeper rings at one workgroup per CU.
constexpr int kG1tD = 3;
// GEMM2's K blocks are half as many bytes of weight per step (bf16 C is the larger operand), so
// four slots still fit two workgroups per CU; D = 4 measured ahead of D = 3 at 2..8 rows/expert.
// 16-row tiles with deeper rings (the freed C space) were slower at 0.5-6 expected rows: D = 5
// and 6 by 1-4% (DS-V3 T=64 126.1 -> 127.9 / 128.2 us), D = 8, one workgroup per CU, by 6-27%.
constexpr int kG2tD = 4;

hipError_t launch_gemm1_tile(const uint8_t* hs, const float* hs_scale, const uint8_t* w13,
                             const float* s13, const int32_t* counts, const int32_t* offsets,
                             const int32_t* sorted_tok, uint16_t* C, int T, int H, int I, int E_l,
                             int max_pairs, hipStream_t stream) {
#define JG_G1T(MT, D)                                                                           \
  {                                                                                             \
    if (H / kBlock < (D) - 1) return hipErrorNotSupported; /* lead must stay within one item */ \
    constexpr int lds = kWaves * D * 2 * kWBlk + D * 16 * MT * kBlock +                         \
                        D * (MT < 4 ? kWave : 16 * MT) * 4 + kWaves * (MT / 2 + 5) * kWave * 4;  \
    const int grid =                                                                            \
        tile_grid(tile_groups_per_cu(lds), tile_count(max_pairs, 16 * MT, E_l) * (I / 64));     \
    gemm1_tile_kernel<MT, D><<<grid, kWaves * kWave, 0, stream>>>(                              \
        hs, hs_scale, w13, s13, counts, offsets, sorted_tok, C, T, H, I, E_l, max_pairs);       \
    return hipGetLastError();                                                                   \
  }
  JG_G1T(2, kG1tD)
#undef JG_G1T
}

hipError_t launch_gemm2_tile(const uint16_t* C, const uint8_t* w2, const float* s2,
                             const int32_t* counts, const int32_t* offsets, const float* sorted_w,
                             Gemm2Out dst, int H, int I, int E_l, int max_pairs, int mt,
                             hipStream_t stream) {
#define JG_G2T(MT, D)                                                                           \
  {                                                                                             \
    if (I / kBlock < (D) - 1 || H % 64 != 0) return hipErrorNotSupported;                      \
    constexpr int lds = kWaves * D * kWBlk + D * 16 * MT * 2 * kBlock +                         \
                        kWaves * (2 * MT + 2) * kWave * 4;                                      \
    const int grid =                                                                            \
        tile_grid(tile_groups_per_cu(lds), tile_count(max_pairs, 16 * MT, E_l) * (H / 64));     \
    gemm2_tile_kernel<MT, D><<<grid, kWaves * kWave, 0, stream>>>(                              \
        C, w2, s2, counts, offsets, sorted_w, dst, H, I, E_l, max_pairs);                       \
    return hipGetLastError();                                                                   \
  }
  if (mt <= 1) JG_G2T(1, kG2tD)
  JG_G2T(2, kG2tD)
#undef JG_G2T
}

}  // namespace jgmoe
