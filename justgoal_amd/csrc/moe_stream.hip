// Weight-streaming grouped GEMMs for small per-expert segments (decode-sized batches).
//
// When an expert holds a handful of pairs, every weight byte feeds at most one 16-row MFMA
// tile, so both GEMMs are HBM streams and the kernels are built around keeping the weight
// stream saturated:
//
// * Work items are per wave: (M-tile of 16*MT pairs, 16 output columns, full K). Each wave loops
//   over its items (persistent grid, items dealt wave-index major); there is no workgroup
//   synchronisation.
// * Weight K-blocks (16 rows x 128 bytes per matrix) go global -> LDS by DMA into a per-wave ring
//   of D slots, two instructions per block, each fetching 8 rows as whole 128-byte lines
//   (register-staged MFMA operands would touch every line twice). The activation rows of the
//   block and its activation scales ride in a matching register ring.
// * The issue side runs D blocks ahead of the compute side and crosses item boundaries: the
//   last D blocks of an item are followed directly by the first D blocks of the wave's next
//   item, so the stream never drains between items. Item metadata (token rows, weight-scale
//   rows) is resolved one item ahead so no load is waited on at an item switch.
// * All waits are counted: each K step issues the same number of vector-memory operations, so
//   "slot d is complete" is vmcnt <= (D-1) * ops_per_step. Blocks past the end of the wave's
//   last item are still issued (to keep that count) but with an out-of-range offset, so they
//   return zeros without fetching anything.
//
// MFMA form: weights are the first operand, so lane l holds output column 4*(l>>4)+i for row
// (pair) l & 15. GEMM1 applies the activation scale (one per lane) times the weight scale of the
// K block after every fp8 MFMA and ends with SwiGLU into bf16 C; GEMM2 converts the fp8 weight
// block to bf16 in registers, runs four bf16 MFMAs per K block over the bf16 C rows, scales by
// the block's weight scale, and stores bf16 rows times the pair's routing weight at the pair's
// destination (the output row for a token's first local pair, else one of its partial rows).
#include "moe_device.h"
#include "moe_kernels.h"


namespace jgmoe {

namespace {

constexpr int kWavesPerGroup = 4;
constexpr int kWBlk = 16 * kBlock;  // one weight K-block image: 16 rows x 128 bytes

// First item of wave w of this workgroup; each wave then takes every (grid * 4)-th item. Wave
// index major: the grid is sized for the most items a batch could have, so when it has fewer
// (one per wave or less: a batch of a few tokens) they still spread over every CU instead of
// filling the first workgroups' four waves and leaving the last CUs idle (DS-V3 T=16: 768 items
// on 256 workgroups of 4 waves used 192 CUs). GEMM1 stage: T=8 30.6 -> 24.0 us, T=16 33.8 ->
// 32.6, T=32 58.7 -> 49.8 (whole call T=8 52.6 -> 46.7, T=32 92.5 -> 83.9).
__device__ __forceinline__ int first_item(int w) { return w * (int)gridDim.x + (int)blockIdx.x; }

// vmcnt holds 6 bits; deeper counts are clamped, which only makes a wait stricter.
constexpr int vm_depth(int n) { return n > 63 ? 63 : n; }

// A per-lane buffer offset past every buffer these kernels address (the API keeps each below
// 2^31 - 16): loads with it return zeros without a memory access.
constexpr uint32_t kNoFetch = 0x7ffffff0u;

// ---- GEMM1: C = SwiGLU(A W1^T, A W3^T) --------------------------------------------------------

template <int MT>
struct G1Slot {
  v8i a[MT];     // activation bytes [32g, 32g+32) of the block for row r16 of each sub-tile
  float sa[MT];  // activation scale of that row and block
};

template <int MT>
struct G1Item {
  const uint8_t* wbase;  // the expert's W13 [2I, H]
  uint32_t wsoff;        // c0 * H: first of the 16 X1 rows
  LaneScales sc1, sc2;   // weight scales of the X1 / X2 row block, per K block
  uint32_t aoff[MT];     // per lane: token * H + 32 g
  uint32_t saoff[MT];    // per lane: token * 4
  int m0, cnt, seg, c0;
};

template <int MT, int D>
__global__ __launch_bounds__(256) void gemm1_stream_kernel(
    const uint8_t* __restrict__ hs, const float* __restrict__ hs_scale,
    const uint8_t* __restrict__ w13, const float* __restrict__ s13,
    const int32_t* __restrict__ counts, const int32_t* __restrict__ offsets,
    const int32_t* __restrict__ sorted_tok, uint16_t* __restrict__ C, int T, int H, int I,
    int E_l) {
  constexpr int BM = 16 * MT;
  constexpr int OPS = 3 * MT + 4;  // vector-memory operations per K step
  __shared__ __attribute__((aligned(16))) uint8_t ring[kWavesPerGroup][D][2 * kWBlk];

  const int lane = threadIdx.x & (kWave - 1), w = wave_id();
  const int r16 = lane & 15, g = lane >> 4;
  const int NCT = I / 16, NKB = H / kBlock;
  TileMap tm;
  tm.init(counts, offsets, E_l, BM);
  const int items = tm.total * NCT;
  const int stride = gridDim.x * kWavesPerGroup;
  int it = __builtin_amdgcn_readfirstlane(first_item(w));
  if (it >= items) return;

  const __amdgpu_buffer_rsrc_t ares = make_rsrc(hs, (uint32_t)T * H);
  const __amdgpu_buffer_rsrc_t sares = make_rsrc(hs_scale, (uint32_t)T * NKB * 4);
  const uint32_t dma0 = wblk_dma_off(lane, 0, H), dma1 = wblk_dma_off(lane, 1, H);
  const uint32_t rd0 = wblk_read_off(lane, 0), rd1 = wblk_read_off(lane, 1);
  uint8_t* my_ring = &ring[w][0][0];

  // Item metadata without the token-dependent offsets; loads the item's token ids into tok.
  auto meta = [&](int item, G1Item<MT>& x, int (&tok)[MT]) {
    item = __builtin_amdgcn_readfirstlane(item);  // keeps the item chain in SGPRs
    const int tile = item / NCT, ct = item % NCT;
    const int e = tm.find(tile, BM, x.m0, x.cnt, x.seg);
    x.c0 = ct * 16;
    x.m0 = uniform(x.m0);
    x.cnt = uniform(x.cnt);
    x.seg = uniform(x.seg);
    x.wbase = uniform(w13 + (size_t)e * 2 * I * H);
    x.wsoff = uniform((uint32_t)x.c0 * H);
    const float* srow = s13 + (size_t)e * (2 * I / kBlock) * NKB;
    x.sc1.load(srow + (size_t)(x.c0 / kBlock) * NKB, NKB);
    x.sc2.load(srow + (size_t)((I + x.c0) / kBlock) * NKB, NKB);
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
      const int r = x.m0 + mt * 16 + r16;
      tok[mt] = sorted_tok[x.seg + (r < x.cnt ? r : x.cnt - 1)];
    }
  };
  auto finish = [&](G1Item<MT>& x, const int (&tok)[MT]) {
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
      x.aoff[mt] = (uint32_t)tok[mt] * H + 32 * g;
      x.saoff[mt] = (uint32_t)tok[mt] * 4;
    }
  };

  G1Item<MT> cur, nxt, nn;
  int tok[MT];
  meta(it, cur, tok);
  finish(cur, tok);
  int it_n = it + stride;
  meta(it_n < items ? it_n : it, nxt, tok);
  finish(nxt, tok);

  G1Slot<MT> sl[D];
  // Issue K block kbi of item cur (or nxt when `second`) into slot d. After a wave's last item
  // there is no next item: those prefetches keep the step's operation count (the counted waits
  // rely on it) but use an out-of-range offset, so they return zeros and fetch nothing.
  auto issue = [&](bool second, int kbi, G1Slot<MT>& s, int d) {
    const bool dead = uniform(second && it_n >= items);
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
      const uint32_t ao = dead ? kNoFetch : second ? nxt.aoff[mt] : cur.aoff[mt];
      const uint32_t so = dead ? kNoFetch : second ? nxt.saoff[mt] : cur.saoff[mt];
      s.a[mt] = buf_load32(ares, ao, (uint32_t)kbi * kBlock);
      s.sa[mt] = __uint_as_float(buf_load32b(sares, so, (uint32_t)kbi * T * 4));
    }
    const __amdgpu_buffer_rsrc_t wres =
        make_rsrc(uniform(second ? nxt.wbase : cur.wbase), 2u * I * H);
    const uint32_t ws = uniform((second ? nxt.wsoff : cur.wsoff) + (uint32_t)kbi * kBlock);
    const uint32_t w0 = dead ? kNoFetch : dma0, w1 = dead ? kNoFetch : dma1;
    uint8_t* slot = my_ring + d * 2 * kWBlk;
    dma16_stream(wres, slot, w0, ws);
    dma16_stream(wres, slot + 1024, w1, ws);
    dma16_stream(wres, slot + kWBlk, w0, ws + (uint32_t)I * H);
    dma16_stream(wres, slot + kWBlk + 1024, w1, ws + (uint32_t)I * H);
  };

  // Prologue in issue order: the loop's wait counts assume every slot's loads went out
  // together, and the loop-entry state would otherwise carry a reordered prologue into them.
#pragma unroll
  for (int d = 0; d < D; ++d) {
    issue(false, d, sl[d], d);
    __builtin_amdgcn_sched_barrier(0);
  }
  retire(nxt.sc1.v0);  // loop entry must not carry pending loads (see the K loop)
  retire(nxt.sc1.v1);
  retire(nxt.sc2.v0);
  retire(nxt.sc2.v1);

  for (;;) {
    // Token ids and scales of the item after nxt, consumed one item from now.
    const int it_nn = it_n + stride;
    meta(it_nn < items ? it_nn : (it_n < items ? it_n : it), nn, tok);

    v4f acc1[MT], acc2[MT];
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
      acc1[mt] = v4f{0.f, 0.f, 0.f, 0.f};
      acc2[mt] = v4f{0.f, 0.f, 0.f, 0.f};
    }
    // do-while: the compiler must see that the trip (with its retires) runs at least once
    int kb0 = 0;
    do {
      const bool last = kb0 + D >= NKB;  // this trip's prefetches belong to the next item
#pragma unroll
      for (int d = 0; d < D; ++d) {
        const int kb = kb0 + d;
        vm_wait<vm_depth((D - 1) * OPS)>();
        const uint32_t base = lds_addr(my_ring + d * 2 * kWBlk);
        v4u x1l = ds_read16(base + rd0), x1h = ds_read16(base + rd1);
        v4u x2l = ds_read16(base + kWBlk + rd0), x2h = ds_read16(base + kWBlk + rd1);
        lds_wait(x1l, x1h, x2l, x2h);
        const v8i b1 = v8i{(int)x1l[0], (int)x1l[1], (int)x1l[2], (int)x1l[3],
                           (int)x1h[0], (int)x1h[1], (int)x1h[2], (int)x1h[3]};
        const v8i b2 = v8i{(int)x2l[0], (int)x2l[1], (int)x2l[2], (int)x2l[3],
                           (int)x2h[0], (int)x2h[1], (int)x2h[2], (int)x2h[3]};
        const float sw1 = cur.sc1.get(kb), sw2 = cur.sc2.get(kb);
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) {
          const float f1 = sl[d].sa[mt] * sw1, f2 = sl[d].sa[mt] * sw2;
          const v4f p = mfma_f8_16x16x128(b1, sl[d].a[mt]);
          const v4f q = mfma_f8_16x16x128(b2, sl[d].a[mt]);
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            acc1[mt][i] = fmaf(p[i], f1, acc1[mt][i]);
            acc2[mt][i] = fmaf(q[i], f2, acc2[mt][i]);
          }
        }
        __builtin_amdgcn_sched_barrier(0);
        issue(last, last ? kb + D - NKB : kb + D, sl[d], d);
        __builtin_amdgcn_sched_barrier(0);
      }
      // The next-but-one item's metadata loads are long complete here; retiring them now
      // keeps their registers' later reuse from waiting on the whole stream.
      retire(nn.sc1.v0);
      retire(nn.sc1.v1);
      retire(nn.sc2.v0);
      retire(nn.sc2.v1);
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) retire(tok[mt]);
      kb0 += D;
    } while (kb0 < NKB);

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
    finish(nxt, tok);
  }
  vm_wait<0>();  // no DMA may still target this workgroup's LDS when it retires
}

// ---- GEMM2: bf16((C W2^T) * routing weight) into the pair's destination row ---------------------

template <int MT>
struct G2Slot {
  uint4 a[MT][4];  // bf16 C values K [32g + 8c, +8) of the block, c < 4, for row r16
};

template <int MT>
struct G2Item {
  const uint8_t* wbase;  // the expert's W2 [H, I]
  uint32_t wsoff;        // h0 * I
  LaneScales sc;         // weight scales of the 128-row block holding h0, per K block
  uint32_t coff[MT];     // per lane: byte offset of C[pair][32 g]
  float wgt[MT];         // routing weight of the lane's pair
  int dst[MT];           // destination row code of the lane's pair (pair_dst)
  int m0, cnt, seg, h0;
};

template <int MT, int D>
__global__ __launch_bounds__(256) void gemm2_stream_kernel(
    const uint16_t* __restrict__ C, const uint8_t* __restrict__ w2, const float* __restrict__ s2,
    const int32_t* __restrict__ counts, const int32_t* __restrict__ offsets,
    const float* __restrict__ sorted_w, Gemm2Out dst, int H, int I, int E_l, int max_pairs) {
  constexpr int BM = 16 * MT;
  constexpr int OPS = 4 * MT + 2;
  __shared__ __attribute__((aligned(16))) uint8_t ring[kWavesPerGroup][D][kWBlk];

  const int lane = threadIdx.x & (kWave - 1), w = wave_id();
  const int r16 = lane & 15, g = lane >> 4;
  const int NHT = H / 16, NKB = I / kBlock;
  TileMap tm;
  tm.init(counts, offsets, E_l, BM);
  const int items = tm.total * NHT;
  const int stride = gridDim.x * kWavesPerGroup;
  int it = __builtin_amdgcn_readfirstlane(first_item(w));
  if (it >= items) return;

  const __amdgpu_buffer_rsrc_t cres = make_rsrc(C, (uint32_t)max_pairs * I * 2);
  const uint32_t dma0 = wblk_dma_off(lane, 0, I), dma1 = wblk_dma_off(lane, 1, I);
  const uint32_t rd0 = wblk_read_off(lane, 0), rd1 = wblk_read_off(lane, 1);
  uint8_t* my_ring = &ring[w][0][0];

  auto meta = [&](int item, G2Item<MT>& x) {
    item = __builtin_amdgcn_readfirstlane(item);
    const int tile = item / NHT, ht = item % NHT;
    const int e = tm.find(tile, BM, x.m0, x.cnt, x.seg);
    x.h0 = ht * 16;
    x.m0 = uniform(x.m0);
    x.cnt = uniform(x.cnt);
    x.seg = uniform(x.seg);
    x.wbase = uniform(w2 + (size_t)e * H * I);
    x.wsoff = uniform((uint32_t)x.h0 * I);
    x.sc.load(s2 + ((size_t)e * (H / kBlock) + x.h0 / kBlock) * NKB, NKB);
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
      const int r = x.m0 + mt * 16 + r16;
      const int p = x.seg + (r < x.cnt ? r : x.cnt - 1);
      x.coff[mt] = ((uint32_t)p * I + 32 * g) * 2;
      x.wgt[mt] = sorted_w[p];
      x.dst[mt] = dst.pair_dst[p];
    }
  };

  G2Item<MT> cur, nxt, nn;
  meta(it, cur);
  int it_n = it + stride;
  meta(it_n < items ? it_n : it, nxt);

  G2Slot<MT> sl[D];
  // As in GEMM1, prefetches past a wave's last item use an out-of-range offset (no traffic).
  auto issue = [&](bool second, int kbi, G2Slot<MT>& s, int d) {
    const bool dead = uniform(second && it_n >= items);
    const __amdgpu_buffer_rsrc_t cr = cres;
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
      const uint32_t co = dead ? kNoFetch : second ? nxt.coff[mt] : cur.coff[mt];
#pragma unroll
      for (int c = 0; c < 4; ++c)
        s.a[mt][c] = buf_load16(cr, co, 2 * (kbi * kBlock + 8 * c));
    }
    const __amdgpu_buffer_rsrc_t wres =
        make_rsrc(uniform(second ? nxt.wbase : cur.wbase), (uint32_t)H * I);
    const uint32_t ws = uniform((second ? nxt.wsoff : cur.wsoff) + (uint32_t)kbi * kBlock);
    uint8_t* slot = my_ring + d * kWBlk;
    dma16_stream(wres, slot, dead ? kNoFetch : dma0, ws);
    dma16_stream(wres, slot + 1024, dead ? kNoFetch : dma1, ws);
  };

  // Prologue in issue order: the loop's wait counts assume every slot's loads went out
  // together, and the loop-entry state would otherwise carry a reordered prologue into them.
#pragma unroll
  for (int d = 0; d < D; ++d) {
    issue(false, d, sl[d], d);
    __builtin_amdgcn_sched_barrier(0);
  }
  retire(nxt.sc.v0);  // loop entry must not carry pending loads (see the K loop)
  retire(nxt.sc.v1);
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) {
    retire(nxt.wgt[mt]);
    retire(nxt.dst[mt]);
  }

  for (;;) {
    const int it_nn = it_n + stride;
    meta(it_nn < items ? it_nn : (it_n < items ? it_n : it), nn);

    v4f acc[MT];
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) acc[mt] = v4f{0.f, 0.f, 0.f, 0.f};
    int kb0 = 0;
    do {
      const bool last = kb0 + D >= NKB;
#pragma unroll
      for (int d = 0; d < D; ++d) {
        const int kb = kb0 + d;
        vm_wait<vm_depth((D - 1) * OPS)>();
        const uint32_t base = lds_addr(my_ring + d * kWBlk);
        v4u lo = ds_read16(base + rd0), hi = ds_read16(base + rd1);
        lds_wait(lo, hi);
        const uint32_t wv[8] = {lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
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
          for (int c = 0; c < 4; ++c)
            t = mfma_bf16_16x16x32(bw[c], __builtin_bit_cast(v8bf, sl[d].a[mt][c]), t);
#pragma unroll
          for (int i = 0; i < 4; ++i) acc[mt][i] = fmaf(t[i], sw, acc[mt][i]);
        }
        __builtin_amdgcn_sched_barrier(0);
        issue(last, last ? kb + D - NKB : kb + D, sl[d], d);
        __builtin_amdgcn_sched_barrier(0);
      }
      retire(nn.sc.v0);
      retire(nn.sc.v1);
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) {
        retire(nn.wgt[mt]);
        retire(nn.dst[mt]);
      }
      kb0 += D;
    } while (kb0 < NKB);

#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
      const int r = cur.m0 + mt * 16 + r16;
      if (r < cur.cnt) {
        const float wp = cur.wgt[mt];
        const int d = cur.dst[mt];
        uint16_t* row = d >= 0 ? dst.out + (size_t)d * H : dst.partial + (size_t)(-1 - d) * H;
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
  vm_wait<0>();
}

}  // namespace

// Persistent grid: `per_cu` workgroups per CU, capped by the largest possible item count.
static int persistent_grid(int per_cu, long long max_items) {
  const int cus = device_cu_count();
  long long g = (long long)cus * per_cu;
  if (g > max_items) g = max_items;
  return g < 1 ? 1 : (int)g;
}

static inline long long max_m_tiles(int max_pairs, int bm, int E_l) {
  return (max_pairs + bm - 1) / bm + (E_l < max_pairs ? E_l : max_pairs);
}

// Workgroups per CU that fit the LDS rings (160 KiB per CU).
static inline int groups_per_cu(int lds_bytes) {
  const int n = (160 * 1024) / lds_bytes;
  return n < 1 ? 1 : n > 8 ? 8 : n;
}

// Ring depth: the largest power of two <= dmax that divides the K-block count, so an item's K
// steps split into whole trips.
static inline int ring_depth(int nkb, int dmax) {
  int d = dmax;
  while (d > 1 && nkb % d != 0) d >>= 1;
  return d;
}

constexpr int kG1StreamD = 8;
constexpr int kG2StreamD = 8;

hipError_t launch_gemm1_stream(const uint8_t* hs, const float* hs_scale, const uint8_t* w13,
                               const float* s13, const int32_t* counts, const int32_t* offsets,
                               const int32_t* sorted_tok, uint16_t* C, int T, int H, int I,
                               int E_l, int max_pairs, int mt, hipStream_t stream) {
  const int nkb = H / kBlock;
#define JG_G1S(MT, D)                                                                          \
  {                                                                                            \
    const long long waves = max_m_tiles(max_pairs, 16 * MT, E_l) * (I / 16);                   \
    const int grid = persistent_grid(groups_per_cu(kWavesPerGroup * D * 2 * kWBlk),            \
                                     (waves + kWavesPerGroup - 1) / kWavesPerGroup);            \
    gemm1_stream_kernel<MT, D><<<grid, kWavesPerGroup * kWave, 0, stream>>>(                   \
        hs, hs_scale, w13, s13, counts, offsets, sorted_tok, C, T, H, I, E_l);                 \
    return hipGetLastError();                                                                  \
  }
  const int d = ring_depth(nkb, mt == 1 ? kG1StreamD : 4);
  if (mt == 1) {
    if (d >= 8) JG_G1S(1, 8)
    if (d == 4) JG_G1S(1, 4)
    if (d == 2) JG_G1S(1, 2)
    JG_G1S(1, 1)
  }
  if (mt == 2) {
    if (d == 4) JG_G1S(2, 4)
    if (d == 2) JG_G1S(2, 2)
    JG_G1S(2, 1)
  }
  if (d == 4) JG_G1S(4, 4)
  if (d == 2) JG_G1S(4, 2)
  JG_G1S(4, 1)
#undef JG_G1S
}

hipError_t launch_gemm2_stream(const uint16_t* C, const uint8_t* w2, const float* s2,
                               const int32_t* counts, const int32_t* offsets,
                               const float* sorted_w, Gemm2Out dst, int H, int I, int E_l,
                               int max_pairs, int mt, hipStream_t stream) {
  const int nkb = I / kBlock;
#define JG_G2S(MT, D)                                                                          \
  {                                                                                            \
    const long long waves = max_m_tiles(max_pairs, 16 * MT, E_l) * (H / 16);                   \
    const int grid = persistent_grid(groups_per_cu(kWavesPerGroup * D * kWBlk),                \
                                     (waves + kWavesPerGroup - 1) / kWavesPerGroup);            \
    gemm2_stream_kernel<MT, D><<<grid, kWavesPerGroup * kWave, 0, stream>>>(                   \
        C, w2, s2, counts, offsets, sorted_w, dst, H, I, E_l, max_pairs);                  \
    return hipGetLastError();                                                                  \
  }
  const int d = ring_depth(nkb, mt == 1 ? kG2StreamD : mt == 2 ? 4 : 2);
  if (mt == 1) {
    if (d >= 8) JG_G2S(1, 8)
    if (d == 4) JG_G2S(1, 4)
    if (d == 2) JG_G2S(1, 2)
    JG_G2S(1, 1)
  }
  if (mt == 2) {
    if (d == 4) JG_G2S(2, 4)
    if (d == 2) JG_G2S(2, 2)
    JG_G2S(2, 1)
  }
  if (d == 2) JG_G2S(4, 2)
  JG_G2S(4, 1)
#undef JG_G2S
}

}  // namespace jgmoe
