// Large-tile grouped GEMMs for longer per-expert segments (GEMM1 from 16 expected pairs per
// expert, GEMM2 from 8; GEMM2's padding-row skip keeps part-filled tiles cheap).
//
// A workgroup (one per CU) computes a 128-row x 128-column output tile of one expert with eight
// compute waves (GEMM1: 2x4 grid, wave tile 64 rows x 32 C columns; GEMM2: 4x2, 32 rows x 64 H
// columns) and one producer wave. Both operands reach LDS by DMA into a 3-slot ring, so every
// weight K-block is fetched once per 128 rows and every activation K-block once per 128
// columns. The same kernels are instantiated with 64-row tiles for shorter segments (2x4 waves
// of 32 x 32; GEMM2 then has room for a 4-slot ring) and, for GEMM1 from 64 to 159 expected
// rows, with four compute waves of 64 x 64; the launchers below pick the form:
//
// * GEMM1: 128 rows of fp8 hidden states (gathered through the pair -> token list) plus their
//   activation scales, and 128 columns of C, i.e. 128 X1 rows and 128 X2 rows of W13. The
//   epilogue applies SwiGLU and stores bf16 C.
// * GEMM2: 128 rows of bf16 C and 128 rows of W2; the epilogue scales by the pair's routing
//   weight and stores bf16 rows at the pair's destination (the token's output row for its first
//   local pair, else one of its partial rows for the combine).
//
// Per K step the producer waits for its own DMAs of the step's block (counted vmcnt), passes the
// workgroup barrier and refills the slot freed by the previous step with the block two steps
// ahead (across item boundaries). The compute waves never touch vector memory in the K loop:
// they read their MFMA fragments from LDS, the next block's first fragments under the current
// block's last MFMAs, with the barrier placed between those two halves. LDS images use XOR
// chunk swizzles chosen for conflict-free ds_read_b128 fragment reads.
#include "moe_device.h"
#include "moe_kernels.h"


namespace jgmoe {

namespace {

constexpr int kWaves = 4;
constexpr int kWBlk = 16 * kBlock;  // 16 rows x 128 bytes

// A buffer offset past every buffer these kernels address (all are < 2 GiB; the launchers check).
constexpr uint32_t kOutOfRange = 0x7ffffff0u;

// Workgroups are dispatched to the 8 XCDs round-robin (workgroup b runs on XCD b % 8), and the
// persistent loop hands workgroup b the items b, b + grid, ... (grid a multiple of 8). This
// bijection on [0, items) gives XCD x a contiguous run of the logical item list instead of
// every 8th item, so consecutive logical items meet in the same L2.
__device__ __forceinline__ int xcd_item(int i, int items) {
  const int x = i & 7, q = items >> 3, r = items & 7;
  return x * q + (x < r ? x : r) + (i >> 3);
}

// Work item -> (expert, first row m0 of its M-tile, N-tile nt). sched bit 0: XCD-contiguous
// physical order (xcd_item); sched >> 1 = GM: 0 = tile-major logical order (the N-tiles of one
// M-tile consecutive), else each expert's M-tiles in bands of GM with the band's items
// N-tile-major (GM M-tiles of one N-tile consecutive).
template <int BM>
__device__ __forceinline__ int map_item(const TileMapLds& tml, int item, int items, int NNT,
                                        int E_l, int sched, int& m0, int& cnt, int& seg,
                                        int& nt) {
  item = uniform((sched & 1) ? xcd_item(item, items) : item);
  const int tile = item / NNT;
  const int e = uniform(tml.template find<BM>(tile, E_l, m0, cnt, seg));
  nt = item - tile * NNT;
  const int GM = sched >> 1;
  if (GM > 0) {
    const int first = tile - uniform(m0) / BM;  // the expert's first tile slot
    const int me = (uniform(cnt) + BM - 1) / BM;
    const int local = item - first * NNT;
    const int band = local / (GM * NNT);
    const int rows = min(GM, me - band * GM);
    const int idx = local - band * GM * NNT;
    nt = idx / rows;
    m0 = (band * GM + idx % rows) * BM;
  }
  nt = uniform(nt);
  return e;
}

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


struct B1Scalars {
  const uint8_t* wbase;  // the expert's W13
  uint32_t c0;           // first C column of the tile
  int e, m0, cnt, seg;
};

// MS: 16-row sub-tiles per compute wave (BM = 32*MS); NS: 16-column sub-tiles (BN = 32*NS).
// MS/NS: 16-row/16-column sub-tiles per compute wave; WM x WN compute waves (wave index w:
// wm = w % WM, wn = w / WM), so BM = 16*MS*WM and BN = 16*NS*WN; wave WM*WN is the producer.
template <int MS, int NS, int D, int WM, int WN>
__global__ __launch_bounds__((WM * WN + 1) * kWave) void gemm1_big_kernel(
    const uint8_t* __restrict__ hs, const float* __restrict__ hs_scale,
    const uint8_t* __restrict__ w13, const float* __restrict__ s13,
    const int32_t* __restrict__ counts, const int32_t* __restrict__ offsets,
    const int32_t* __restrict__ sorted_tok, uint16_t* __restrict__ C, int T, int H, int I,
    int E_l, int max_pairs, int sched) {
  static_assert(D >= 3, "the prefetch lead is D-1 blocks");
  static_assert(16 * NS <= kBlock && kBlock % (16 * NS) == 0, "a wave's columns share one scale block");
  constexpr int BM = 16 * MS * WM, BN = 16 * NS * WN;
  constexpr int kComputeWaves = WM * WN, kProducer = WM * WN;
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
  __shared__ TileMapLds tml;
  const int items = uniform(tml.build(counts, offsets, E_l, BM, w == 0)) * NNT;
  int it = uniform((int)blockIdx.x);
  if (it >= items) return;  // whole workgroup
  __syncthreads();  // whole workgroup
  const int stride = gridDim.x;

  auto scalars = [&](int item, B1Scalars& x) {
    int nt;
    x.e = uniform(map_item<BM>(tml, item, items, NNT, E_l, sched, x.m0, x.cnt, x.seg, nt));
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
      // Rows past the segment get an offset beyond both buffers: their DMAs fetch nothing (the
      // LDS rows they would fill only feed output rows that are never stored).
      const int valid = x.s.cnt - x.s.m0;
#pragma unroll
      for (int j = 0; j < AI; ++j)
        x.aoff[j] = 8 * j + (lane >> 3) < valid
                        ? __float_as_uint(t[j]) * H + 16 * ((lane & 7) ^ wblk_swz(8 * j + (lane >> 3)))
                        : kOutOfRange;
#pragma unroll
      for (int k = 0; k < SI; ++k)
        x.saoff[k] = k * kWave + lane < valid ? __float_as_uint(t[AI + k]) * 4 : kOutOfRange;
    };
    P cur, nxt, nn;
    meta(it, cur);
    vm_wait<0>();
    finish(cur);
    meta(it_n < items ? it_n : it, nxt);
    vm_wait<0>();
    finish(nxt);

    auto issue = [&](const P& x, int kbi, int slot) {
#pragma unroll
      for (int j = 0; j < AI; ++j)
        dma16(ares, &aring[slot][j * 1024], x.aoff[j],
              (uint32_t)kbi * kBlock);
#pragma unroll
      for (int k = 0; k < SI; ++k)
        dma4(sares, &sring[slot][k * kWave], x.saoff[k],
             (uint32_t)kbi * T * 4);
      const __amdgpu_buffer_rsrc_t wres = make_rsrc(uniform(x.s.wbase), 2u * I * H);
      const uint32_t c0 = uniform(x.s.c0);
      // An expert with a single M-tile reads each W13 byte once per call: its weight DMAs carry
      // the non-temporal hint; experts with more M-tiles share their weight tiles in L2.
      if (uniform(x.s.cnt) <= BM) {
#pragma unroll
        for (int j = 0; j < BI; ++j) {
          const int grp = j >> 1;
          const uint32_t row0 = grp < BN / 16 ? c0 + 16 * grp : I + c0 + 16 * (grp - BN / 16);
          dma16_stream(wres, &bring[slot][j * 1024], (j & 1) ? dma1 : dma0,
                       uniform(row0 * H + (uint32_t)kbi * kBlock));
        }
      } else {
#pragma unroll
        for (int j = 0; j < BI; ++j) {
          const int grp = j >> 1;
          const uint32_t row0 = grp < BN / 16 ? c0 + 16 * grp : I + c0 + 16 * (grp - BN / 16);
          dma16(wres, &bring[slot][j * 1024], (j & 1) ? dma1 : dma0,
                uniform(row0 * H + (uint32_t)kbi * kBlock));
        }
      }
    };
#pragma unroll
    for (int d = 0; d < D - 1; ++d) {
      issue(cur, d, d);
      __builtin_amdgcn_sched_barrier(0);
    }
    int slot = 0;
    for (;;) {
      const int it_nn = it_n + stride;
      meta(it_nn < items ? it_nn : (it_n < items ? it_n : it), nn);
      // Refills come from the current item until its last block is issued, then from the next
      // one; two loops (not a per-step select) so the current item's offsets are dead in the
      // second and only two items' offsets are ever live.
      int kb = 0;
      for (; kb + D - 1 < NKB; ++kb) {
        vm_wait<vm_depth((D - 2) * OPS)>();  // the DMAs of block kb have landed
        __builtin_amdgcn_s_barrier();
        issue(cur, kb + D - 1, slot == 0 ? D - 1 : slot - 1);
        __builtin_amdgcn_sched_barrier(0);
        slot = slot + 1 == D ? 0 : slot + 1;
      }
      for (; kb < NKB; ++kb) {
        vm_wait<vm_depth((D - 2) * OPS)>();
        __builtin_amdgcn_s_barrier();
        issue(nxt, kb + D - 1 - NKB, slot == 0 ? D - 1 : slot - 1);
        __builtin_amdgcn_sched_barrier(0);
        slot = slot + 1 == D ? 0 : slot + 1;
      }
      vm_wait<vm_depth((D - 1) * OPS)>();  // the token-list DMAs of the next-but-one tile
      finish(nn);
      if (it_n >= items) break;
      it = it_n;
      it_n = it_nn;
      cur = nxt;
      nxt = nn;
    }
    __builtin_amdgcn_s_barrier();  // pairs with the compute waves' barrier after their last block
    vm_wait<0>();  // no DMA may still target this workgroup's LDS when it retires
    return;
  }

  // ---------------- compute waves ----------------
  const int wm = w % WM, wn = w / WM;
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

  // Software pipeline. The fragments a step needs first (A sub-tiles 0 and 1, the first column
  // sub-tile of B, the activation scales) are read during the previous step; the remaining A
  // sub-tiles are read under the first column sub-tile's MFMAs and each further B column
  // sub-tile under the previous one's. The step's barrier for the next block sits between the
  // two MFMA halves of the last column sub-tile, when every read of the current slot is done.
  static_assert(MS >= 2 && NS % 2 == 0, "pipeline shape");
  v4u al[MS], ah[MS];  // A fragments of the step, per 16-row sub-tile
  v4u bq[2][4];        // B fragments (X1 lo/hi, X2 lo/hi) of two column sub-tiles
  float sa[MS];        // activation scales of the lane's rows
  auto a_base = [&](int d) { return lds_addr(&aring[d][0]) + wm * MS * kWBlk; };
  auto b_base = [&](int d) { return lds_addr(&bring[d][0]) + wn * NS * kWBlk; };
  auto read_a = [&](uint32_t ab, int ms) {
    al[ms] = ds_read16(ab + ms * kWBlk + rd0);
    ah[ms] = ds_read16(ab + ms * kWBlk + rd1);
  };
  auto read_b = [&](uint32_t bb, int ns, v4u(&b)[4]) {
    b[0] = ds_read16(bb + ns * kWBlk + rd0);
    b[1] = ds_read16(bb + ns * kWBlk + rd1);
    b[2] = ds_read16(bb + (BN / 16 + ns) * kWBlk + rd0);
    b[3] = ds_read16(bb + (BN / 16 + ns) * kWBlk + rd1);
  };
  auto read_head = [&](int d) {  // what the first MFMAs of a step need
    const uint32_t ab = a_base(d);
    read_a(ab, 0);
    read_a(ab, 1);
    read_b(b_base(d), 0, bq[0]);
    const uint32_t sb = lds_addr(&sring[d][0]) + 4 * (wm * MS * 16 + r16);
#pragma unroll
    for (int ms = 0; ms < MS; ++ms) sa[ms] = ds_read4f(sb + 4 * 16 * ms);
  };
  auto fence_a = [&](int ms) {
    lds_fence(al[ms]);
    lds_fence(ah[ms]);
  };
  auto fence_b = [&](v4u(&b)[4]) {
#pragma unroll
    for (int i = 0; i < 4; ++i) lds_fence(b[i]);
  };

  int slot = 0;
  __builtin_amdgcn_s_barrier();  // block 0 has landed
  read_head(0);
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
      const int d = slot, dn = slot + 1 == D ? 0 : slot + 1;
      const uint32_t ab = a_base(d), bb = b_base(d);
      const float sw1 = cur.sc1.get(kb), sw2 = cur.sc2.get(kb);
      lds_wait_all();  // the head fragments (read during the previous step) have landed
      fence_a(0);
      fence_a(1);
      fence_b(bq[0]);
      float f1[MS], f2[MS];
#pragma unroll
      for (int ms = 0; ms < MS; ++ms) {
        lds_fence(sa[ms]);
        f1[ms] = sa[ms] * sw1;
        f2[ms] = sa[ms] * sw2;
      }
      auto mma = [&](int ms, int ns, const v4u(&b)[4]) {
        const v8i a = v8i{(int)al[ms][0], (int)al[ms][1], (int)al[ms][2], (int)al[ms][3],
                          (int)ah[ms][0], (int)ah[ms][1], (int)ah[ms][2], (int)ah[ms][3]};
        const v8i b1 = v8i{(int)b[0][0], (int)b[0][1], (int)b[0][2], (int)b[0][3],
                           (int)b[1][0], (int)b[1][1], (int)b[1][2], (int)b[1][3]};
        const v8i b2 = v8i{(int)b[2][0], (int)b[2][1], (int)b[2][2], (int)b[2][3],
                           (int)b[3][0], (int)b[3][1], (int)b[3][2], (int)b[3][3]};
        const v4f p = mfma_f8_16x16x128(b1, a);
        const v4f q = mfma_f8_16x16x128(b2, a);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          acc1[ms][ns][i] = fmaf(p[i], f1[ms], acc1[ms][ns][i]);
          acc2[ms][ns][i] = fmaf(q[i], f2[ms], acc2[ms][ns][i]);
        }
      };
      // column sub-tile 0: the other A sub-tiles and B column sub-tile 1 arrive meanwhile
#pragma unroll
      for (int ms = 2; ms < MS; ++ms) read_a(ab, ms);
      read_b(bb, 1, bq[1]);
      mma(0, 0, bq[0]);
      mma(1, 0, bq[0]);
      lds_wait_all();
#pragma unroll
      for (int ms = 2; ms < MS; ++ms) fence_a(ms);
      fence_b(bq[1]);
#pragma unroll
      for (int ms = 2; ms < MS; ++ms) mma(ms, 0, bq[0]);
#pragma unroll
      for (int ns = 1; ns < NS; ++ns) {
        v4u(&b)[4] = bq[ns & 1];
        if (ns + 1 < NS) {
          read_b(bb, ns + 1, bq[(ns + 1) & 1]);
#pragma unroll
          for (int ms = 0; ms < MS; ++ms) mma(ms, ns, b);
          lds_wait_all();
          fence_b(bq[(ns + 1) & 1]);
        } else {
          // last column sub-tile (bq[1]; bq[0] is free for the next block's head)
          mma(0, ns, b);
          mma(1, ns, b);
          // Block kb+1 has landed and slot d is no longer read. After the last block this
          // barrier pairs with the producer's final one and the head read is unused.
          __builtin_amdgcn_s_barrier();
          read_head(dn);
          __builtin_amdgcn_sched_barrier(0);  // keep the head reads ahead of the last MFMAs
#pragma unroll
          for (int ms = 2; ms < MS; ++ms) mma(ms, ns, b);
        }
      }
      slot = dn;
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

// MS/NS: 16-row/16-column sub-tiles per compute wave; WM x WN compute waves (wave index w:
// wm = w / WN, wn = w % WN), so BM = 16*MS*WM and BN = 16*NS*WN; wave WM*WN is the producer.
template <int MS, int NS, int D, int WM, int WN>
__global__ __launch_bounds__((WM * WN + 1) * kWave) void gemm2_big_kernel(
    const uint16_t* __restrict__ C, const uint8_t* __restrict__ w2, const float* __restrict__ s2,
    const int32_t* __restrict__ counts, const int32_t* __restrict__ offsets,
    const float* __restrict__ sorted_w, Gemm2Out dst, int H, int I, int E_l, int max_pairs,
    int sched) {
  static_assert(D >= 3, "the prefetch lead is D-1 blocks");
  static_assert(16 * NS <= kBlock && kBlock % (16 * NS) == 0, "a wave's columns share one scale block");
  constexpr int BM = 16 * MS * WM, BN = 16 * NS * WN;
  constexpr int kComputeWaves = WM * WN, kProducer = WM * WN;
  constexpr int ARow = 2 * kBlock;    // bf16 C bytes per row per K block
  constexpr int AI = BM / 4;          // C DMA instructions per step (4 rows x 256 B each)
  constexpr int BI = BN / 8;          // W2 DMA instructions per step (8 rows x 128 B each)
  constexpr int OPS = AI + BI;
  constexpr int MW = 2 * MS + 2;      // compute-wave metadata dwords per lane
  constexpr int ASZ = BM * ARow, BSZ = BN * kBlock;
  __shared__ __attribute__((aligned(16))) uint8_t aring[D][ASZ];
  __shared__ __attribute__((aligned(16))) uint8_t bring[D][BSZ];
  __shared__ __attribute__((aligned(16))) float mring[kComputeWaves][MW][kWave];

  const int lane = threadIdx.x & (kWave - 1), w = wave_id();
  const int NNT = H / BN, NKB = I / kBlock;
  __shared__ TileMapLds tml;
  const int items = uniform(tml.build(counts, offsets, E_l, BM, w == 0)) * NNT;
  int it = uniform((int)blockIdx.x);
  if (it >= items) return;  // whole workgroup
  __syncthreads();
  const int stride = gridDim.x;

  auto scalars = [&](int item, B2Scalars& x) {
    int nt;
    x.e = uniform(map_item<BM>(tml, item, items, NNT, E_l, sched, x.m0, x.cnt, x.seg, nt));
    x.m0 = uniform(x.m0);
    x.cnt = uniform(x.cnt);
    x.seg = uniform(x.seg);
    x.h0 = uniform((uint32_t)(nt * BN));
    x.wbase = uniform(w2 + (size_t)x.e * H * I);
  };
  int it_n = it + stride;

  if (w == kProducer) {
    const uint32_t dma0 = wblk_dma_off(lane, 0, I), dma1 = wblk_dma_off(lane, 1, I);
    // C DMA instruction j covers tile rows 4j + lane/16, chunk position lane & 15 holding
    // chunk (lane & 15) ^ crow_swz(row). The offsets are relative to the tile's first row and the
    // same for every item: each item's buffer resource starts at that row and ends at the
    // segment's last row, so rows past the segment are out of range (never fetched).
    uint32_t aoff[AI];
#pragma unroll
    for (int j = 0; j < AI; ++j) {
      const int row = 4 * j + (lane >> 4);
      aoff[j] = (uint32_t)row * I * 2 + 16 * ((lane & 15) ^ crow_swz(row));
    }
    B2Scalars cur, nxt, nn;
    scalars(it, cur);
    scalars(it_n < items ? it_n : it, nxt);
    auto issue = [&](bool second, int kbi, int slot) {
      const B2Scalars& x = second ? nxt : cur;
      const int m0 = uniform(x.m0);
      const __amdgpu_buffer_rsrc_t cres =
          make_rsrc(uniform(C + (size_t)(uniform(x.seg) + m0) * I),
                    uniform((uint32_t)(uniform(x.cnt) - m0) * I * 2));
#pragma unroll
      for (int j = 0; j < AI; ++j)
        dma16(cres, &aring[slot][j * 1024], aoff[j], (uint32_t)kbi * ARow);
      const __amdgpu_buffer_rsrc_t wres = make_rsrc(uniform(x.wbase), (uint32_t)H * I);
      const uint32_t h0 = uniform(x.h0);
      // as in GEMM1: non-temporal weight DMAs for experts with a single M-tile
      if (uniform(x.cnt) <= BM) {
#pragma unroll
        for (int j = 0; j < BI; ++j)
          dma16_stream(wres, &bring[slot][j * 1024], (j & 1) ? dma1 : dma0,
                       uniform((h0 + 16 * (j >> 1)) * (uint32_t)I + (uint32_t)kbi * kBlock));
      } else {
#pragma unroll
        for (int j = 0; j < BI; ++j)
          dma16(wres, &bring[slot][j * 1024], (j & 1) ? dma1 : dma0,
                uniform((h0 + 16 * (j >> 1)) * (uint32_t)I + (uint32_t)kbi * kBlock));
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
      scalars(it_nn < items ? it_nn : (it_n < items ? it_n : it), nn);
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
    __builtin_amdgcn_s_barrier();  // pairs with the compute waves' barrier after their last block
    vm_wait<0>();
    return;
  }

  // Row-major wave order (w = wm*WN + wn): the two compute waves that share a SIMD (w and w+4)
  // hold row slices wm and wm+2, so the all-padding slices of a part-filled tile (which skip
  // their MFMAs below) spread over the SIMDs instead of idling some while others carry two.
  const int wm = w / WN, wn = w % WN;
  const int r16 = lane & 15, g = lane >> 4;
  const __amdgpu_buffer_rsrc_t wgtres = make_rsrc(sorted_w, (uint32_t)max_pairs * 4);
  const __amdgpu_buffer_rsrc_t dstres = make_rsrc(dst.pair_dst, (uint32_t)max_pairs * 4);
  const __amdgpu_buffer_rsrc_t s2res = make_rsrc(s2, (uint32_t)E_l * (H / kBlock) * NKB * 4);
  const uint32_t rd0 = wblk_read_off(lane, 0), rd1 = wblk_read_off(lane, 1);
  float* my_meta = &mring[w][0][0];
  struct Q {
    B2Scalars s;
    LaneScales sc;  // weight scales of this wave's columns (one 128-block)
    float wgt[MS];  // routing weight of the lane's output row in each sub-tile
    int dst[MS];    // destination row code (pair_dst) of that row
  };
  auto meta = [&](int item, Q& x) {
    scalars(item, x.s);
    const int last = x.s.cnt - 1;
#pragma unroll
    for (int ms = 0; ms < MS; ++ms) {
      const int r = x.s.m0 + (wm * MS + ms) * 16 + r16;
      dma4(wgtres, my_meta + ms * kWave, 4u * (x.s.seg + (r < last ? r : last)), 0);
      dma4(dstres, my_meta + (MS + 2 + ms) * kWave, 4u * (x.s.seg + (r < last ? r : last)), 0);
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
    for (int ms = 0; ms < MS; ++ms) {
      x.wgt[ms] = v[ms];
      x.dst[ms] = __float_as_int(v[MS + 2 + ms]);
    }
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

  // Software pipeline (rows outer): the W2 fragments of a step and its first C sub-tile are read
  // during the previous step, C sub-tile ms+1 under sub-tile ms's MFMAs; the barrier for the
  // next block sits between the two MFMA halves of the last row sub-tile.
  static_assert(MS % 2 == 0 && NS % 2 == 0, "pipeline shape");
  v4u wq[NS][2];  // raw e4m3 W2 fragments of the step
  v4u a[2][4];    // C fragments of two row sub-tiles
  auto read_a = [&](uint32_t ab, int ms, v4u(&x)[4]) {
    const int row = (wm * MS + ms) * 16 + r16;
#pragma unroll
    for (int c = 0; c < 4; ++c) x[c] = ds_read16(ab + row * ARow + 16 * ((4 * g + c) ^ crow_swz(row)));
  };
  auto read_head = [&](int d) {
    const uint32_t bb = lds_addr(&bring[d][0]) + wn * NS * kWBlk;
#pragma unroll
    for (int ns = 0; ns < NS; ++ns) {
      wq[ns][0] = ds_read16(bb + ns * kWBlk + rd0);
      wq[ns][1] = ds_read16(bb + ns * kWBlk + rd1);
    }
    read_a(lds_addr(&aring[d][0]), 0, a[0]);
  };

  int slot = 0;
  __builtin_amdgcn_s_barrier();  // block 0 has landed
  read_head(0);
  for (;;) {
    const int it_nn = it_n + stride;
    meta(it_nn < items ? it_nn : (it_n < items ? it_n : it), nn);
    v4f acc[MS][NS];
#pragma unroll
    for (int ms = 0; ms < MS; ++ms)
#pragma unroll
      for (int ns = 0; ns < NS; ++ns) acc[ms][ns] = v4f{0.f, 0.f, 0.f, 0.f};
    // A wave whose 16*MS rows of the tile are all padding only keeps the workgroup's per-step
    // barriers and reads the next item's head at its last step.
    const bool busy = cur.s.m0 + wm * MS * 16 < cur.s.cnt;
    // The head fragments come from asm LDS reads that the compiler takes as complete at once;
    // where the two loop forms join it may copy them, so both forms wait for them first.
    auto fence_head = [&] {
      lds_wait_all();
#pragma unroll
      for (int ns = 0; ns < NS; ++ns) {
        lds_fence(wq[ns][0]);
        lds_fence(wq[ns][1]);
      }
#pragma unroll
      for (int c = 0; c < 4; ++c) lds_fence(a[0][c]);
    };
    if (!busy) {
      int kb = 0;
      do {
        const int dn = slot + 1 == D ? 0 : slot + 1;
        lds_wait_all();
        __builtin_amdgcn_s_barrier();
        if (kb + 1 == NKB) read_head(dn);
        slot = dn;
        ++kb;
      } while (kb < NKB);
      fence_head();
    } else {
      int kb = 0;
      do {
        const int d = slot, dn = slot + 1 == D ? 0 : slot + 1;
        const uint32_t ab = lds_addr(&aring[d][0]);
        const float sw = cur.sc.get(kb);
        lds_wait_all();  // the head fragments have landed
        v8bf bw[NS][4];
#pragma unroll
        for (int ns = 0; ns < NS; ++ns) {
          lds_fence(wq[ns][0]);
          lds_fence(wq[ns][1]);
          const uint32_t wv[8] = {wq[ns][0][0], wq[ns][0][1], wq[ns][0][2], wq[ns][0][3],
                                  wq[ns][1][0], wq[ns][1][1], wq[ns][1][2], wq[ns][1][3]};
#pragma unroll
          for (int c = 0; c < 4; ++c) {
            v2bf p0, p1, p2, p3;
            fp8x4_to_bf16x4((int)wv[2 * c], p0, p1);
            fp8x4_to_bf16x4((int)wv[2 * c + 1], p2, p3);
            bw[ns][c] = v8bf{p0[0], p0[1], p1[0], p1[1], p2[0], p2[1], p3[0], p3[1]};
          }
        }
#pragma unroll
        for (int c = 0; c < 4; ++c) lds_fence(a[0][c]);
        // Column sub-tiles [n0, n1) of row sub-tile ms, their four K-chunk MFMAs interleaved
        // (chunk outer) so that consecutive MFMAs are independent (chained per sub-tile they
        // measured 2% slower), then the s2 block scale.
        auto mma_row = [&](int ms, int n0, int n1, const v4u(&x)[4]) {
          v4f t[NS];
#pragma unroll
          for (int ns = 0; ns < NS; ++ns) t[ns] = v4f{0.f, 0.f, 0.f, 0.f};
#pragma unroll
          for (int c = 0; c < 4; ++c)
#pragma unroll
            for (int ns = n0; ns < n1; ++ns)
              t[ns] = mfma_bf16_16x16x32(bw[ns][c], __builtin_bit_cast(v8bf, x[c]), t[ns]);
#pragma unroll
          for (int ns = n0; ns < n1; ++ns)
#pragma unroll
            for (int i = 0; i < 4; ++i) acc[ms][ns][i] = fmaf(t[ns][i], sw, acc[ms][ns][i]);
        };
#pragma unroll
        for (int ms = 0; ms < MS; ++ms) {
          v4u(&x)[4] = a[ms & 1];
          if (ms + 1 < MS) {
            read_a(ab, ms + 1, a[(ms + 1) & 1]);
            mma_row(ms, 0, NS, x);
            lds_wait_all();
#pragma unroll
            for (int c = 0; c < 4; ++c) lds_fence(a[(ms + 1) & 1][c]);
          } else {
            // last row sub-tile (a[1]; a[0] and wq are free for the next block's head)
            mma_row(ms, 0, NS / 2, x);
            // Block kb+1 has landed and slot d is no longer read. After the last block this
            // barrier pairs with the producer's final one and the head read is unused.
            __builtin_amdgcn_s_barrier();
            read_head(dn);  // (pinning these ahead of the MFMAs, as in GEMM1, measured slower here)
            mma_row(ms, NS / 2, NS, x);
          }
        }
        slot = dn;
        ++kb;
      } while (kb < NKB);
      fence_head();
    }
    vm_wait<0>();
    finish(nn);

#pragma unroll
    for (int ms = 0; ms < MS; ++ms) {
      const int r = cur.s.m0 + (wm * MS + ms) * 16 + r16;
      if (r < cur.s.cnt) {
        const float wp = cur.wgt[ms];
        const int d = cur.dst[ms];
        uint16_t* orow = (d >= 0 ? dst.out + (size_t)d * H : dst.partial + (size_t)(-1 - d) * H) +
                         cur.s.h0 + wn * 16 * NS + 4 * g;
#pragma unroll
        for (int ns = 0; ns < NS; ++ns) {
          const uint32_t h01 = (uint32_t)float_to_bf16_bits(acc[ms][ns][0] * wp) |
                               ((uint32_t)float_to_bf16_bits(acc[ms][ns][1] * wp) << 16);
          const uint32_t h23 = (uint32_t)float_to_bf16_bits(acc[ms][ns][2] * wp) |
                               ((uint32_t)float_to_bf16_bits(acc[ms][ns][3] * wp) << 16);
          *(uint2*)(orow + 16 * ns) = uint2{h01, h23};
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

}  // namespace

// Item schedules (map_item). The banded one: XCD-contiguous physical order over bands of 8
// M-tiles, N-tile-major inside a band, so an XCD's 32 concurrent items share W13 panels across
// up to 8 M-tiles and activation rows across 4 N-tiles. For GEMM1 it fetches fewer bytes than
// the tile-major round-robin order (T=4096: 0.89 against 1.19 GB, algorithmic 0.80; T=16384
// skewed: 6.07 against 7.96 GB) and made the Qwen3-style T=1024 batch's GEMM1 364 -> 327 us.
// GEMM2 keeps the tile-major round-robin order: every variant tried (XCD-contiguous, bands of
// 2-16) was 1-5% slower there.
constexpr int kSchedGemm1 = 1 | (8 << 1);
constexpr int kSchedGemm2 = 0;
// Tile-major round-robin puts item i on XCD i % 8. When an expert has a multiple of 8 N-tiles,
// each weight panel (expert, N-tile) then stays on one XCD for all of the expert's M-tiles, and
// that order beats the banded XCD-contiguous one: DS-V3 GEMM1 (16 N-tiles) T=768 124.7 -> 123.0
// us, T=1024 130.3 -> 125.1, T=1536 164.2 -> 158.5, T=2048 150.0 -> 141.3, T=3072 195.9 -> 182.1,
// T=4096 204.5 -> 202.0, T=16384 skewed 1939 -> 1910. With 12 N-tiles (Qwen3-style GEMM1)
// round-robin scatters each panel and each expert's activation rows over the XCDs and is 7-13%
// slower (T=512 286 -> 324, T=1024 305 -> 345 us), so the banded order stays there. GEMM2 (56 or
// 32 N-tiles) always has a multiple of 8.
constexpr int kXcds = 8;
constexpr int gemm1_sched(int n_tiles) { return n_tiles % kXcds == 0 ? 0 : kSchedGemm1; }

static int big_grid(long long max_items) {
  const int cus = device_cu_count();
  long long g = cus;  // the LDS rings leave room for one workgroup per CU
  if (g > max_items) g = max_items;
  return g < 1 ? 1 : (int)g;
}

static inline long long big_tiles(int max_pairs, int bm, int E_l) {
  return (max_pairs + bm - 1) / bm + (E_l < max_pairs ? E_l : max_pairs);
}

constexpr int kB1Ms = 4;
constexpr int kB1Ns = 2;
constexpr int kB1Wm = 2;
constexpr int kB1Wn = 4;
constexpr int kB1D = 3;
// GEMM1 for 16..63 expected rows per expert: 64-row tiles (MS = 2, wave tile 32 rows x 32 C
// columns; 40 KB of DMA per K step for 4.2 MFLOP per CU against 48 KB in the two 64-row
// workgroups per CU of the LDS-tiled kernel), results bit-identical. Whole call against the
// LDS-tiled GEMM1, two weight sets in rotation: DS-V3 T=512 211.3 -> 204.4 us, T=768 237.0 ->
// 218.8, T=1024 249.8 -> 232.1, T=1536 309.9 -> 285.6, T=1792 343.7 -> 294.9; Qwen3-style T=256
// 446.4 -> 427.9, T=512 485.5 -> 473.2, T=768 536.5 -> 517.9. Below 16 rows DS-V3 is slower on
// them (T=256 171.1 against 187.9), and from 64 the 128-row tiles stay ahead (T=2048 301.8
// against 307.7, T=4096 428.2 against 469.9).
constexpr int kB1TallRows = 64;
constexpr int kB1ShortMs = 2;
// 128-row tiles below 160 expected rows: 4 compute waves of 64 rows x 64 C columns (2 x 2; five
// waves per workgroup, so up to 256 VGPRs each, and a quarter less LDS fragment traffic per K
// step) instead of 8 of 64 x 32. Bit-identical; GEMM1 stage against the 8-wave form, both on
// the item order of gemm1_sched: DS-V3 T=2048 146.4 -> 142.0 us, T=3072 185.8 -> 182.9, T=4096
// 202.9 -> 201.4; Qwen3-style T=1024 321 -> 307 (banded order), T=1536 334.3 -> 325.1, T=2048
// 382.3 -> 371.0. From 160 rows, where GEMM1 turns MFMA-bound, the 8-wave form, whose two waves
// per SIMD overlap one's MFMAs with the other's scale FMAs, is ahead: T=5120 235.2 against
// 240.9, T=6144 248.7 against 256.6, T=8192 334.5 against 341.3, T=16384 skewed 1922 against
// 2006. The same 2 x 2 layout measured within 1% for the 64-row tiles of both GEMMs, and 4-8%
// slower for GEMM2's 128-row tiles (2 x 2, or 4 x 1 waves of 32 x 128) at T=2048-16384.
constexpr int kB1EightWaveRows = 160;
constexpr int kB1WideNs = 4;
constexpr int kB1WideWm = 2;
constexpr int kB1WideWn = 2;
constexpr int kB2Ms = 2;
constexpr int kB2Ns = 4;
constexpr int kB2Wm = 4;
constexpr int kB2Wn = 2;
constexpr int kB2D = 3;
// GEMM2 for 8..63 expected rows per expert: 64-row tiles (2 x 4 waves of 32 x 32, NS = 2) in a
// 4-slot ring (146 KB of LDS). Against the 128-row tiles, whole call, two weight sets in
// rotation, results bit-identical: DS-V3 T=768 252.1 -> 236.6 us, T=1024 260.6 -> 249.8,
// T=1280 283.0 -> 275.4, T=1536 310.0 -> 306.9, T=1792 344.1 -> 339.9; Qwen3-style T=512 503.3 ->
// 486.0, T=640 515.0 -> 504.0, T=768 541.2 -> 534.4. From 64 rows the 128-row tiles stay ahead
// (DS-V3 T=2048 299.8 against 304.6, Qwen3-style T=1024 554.0 against 568.4). A 3-slot ring
// was 0.4-1.5% behind the 4-slot one everywhere.
constexpr int kB2TallRows = 64;
constexpr int kB2ShortWm = 2;
constexpr int kB2ShortWn = 4;
constexpr int kB2ShortNs = 2;
constexpr int kB2ShortD = 4;

template <int MS, int NS, int D, int WM, int WN>
static hipError_t launch_gemm1_big_t(const uint8_t* hs, const float* hs_scale, const uint8_t* w13,
                                     const float* s13, const int32_t* counts,
                                     const int32_t* offsets, const int32_t* sorted_tok,
                                     uint16_t* C, int T, int H, int I, int E_l, int max_pairs,
                                     hipStream_t stream) {
  constexpr int BN = 16 * NS * WN;
  if (I % BN != 0 || H / kBlock < D - 1 || (int64_t)T * H >= kOutOfRange)
    return hipErrorNotSupported;
  const int grid = big_grid(big_tiles(max_pairs, 16 * MS * WM, E_l) * (I / BN));
  gemm1_big_kernel<MS, NS, D, WM, WN><<<grid, (WM * WN + 1) * kWave, 0, stream>>>(
      hs, hs_scale, w13, s13, counts, offsets, sorted_tok, C, T, H, I, E_l, max_pairs,
      gemm1_sched(I / BN));
  return hipGetLastError();
}

hipError_t launch_gemm1_big(const uint8_t* hs, const float* hs_scale, const uint8_t* w13,
                            const float* s13, const int32_t* counts, const int32_t* offsets,
                            const int32_t* sorted_tok, uint16_t* C, int T, int H, int I, int E_l,
                            int max_pairs, int rows_hint, hipStream_t stream) {
  if (rows_hint < kB1TallRows)
    return launch_gemm1_big_t<kB1ShortMs, kB1Ns, kB1D, kB1Wm, kB1Wn>(
        hs, hs_scale, w13, s13, counts, offsets, sorted_tok, C, T, H, I, E_l, max_pairs, stream);
  if (rows_hint < kB1EightWaveRows)
    return launch_gemm1_big_t<kB1Ms, kB1WideNs, kB1D, kB1WideWm, kB1WideWn>(
        hs, hs_scale, w13, s13, counts, offsets, sorted_tok, C, T, H, I, E_l, max_pairs, stream);
  return launch_gemm1_big_t<kB1Ms, kB1Ns, kB1D, kB1Wm, kB1Wn>(hs, hs_scale, w13, s13, counts,
                                                              offsets, sorted_tok, C, T, H, I,
                                                              E_l, max_pairs, stream);
}

template <int MS, int NS, int D, int WM, int WN>
static hipError_t launch_gemm2_big_t(const uint16_t* C, const uint8_t* w2, const float* s2,
                                     const int32_t* counts, const int32_t* offsets,
                                     const float* sorted_w, Gemm2Out dst, int H, int I, int E_l,
                                     int max_pairs, hipStream_t stream) {
  constexpr int BN = 16 * NS * WN;
  if (H % BN != 0 || I / kBlock < D - 1) return hipErrorNotSupported;
  const int grid = big_grid(big_tiles(max_pairs, 16 * MS * WM, E_l) * (H / BN));
  gemm2_big_kernel<MS, NS, D, WM, WN><<<grid, (WM * WN + 1) * kWave, 0, stream>>>(
      C, w2, s2, counts, offsets, sorted_w, dst, H, I, E_l, max_pairs, kSchedGemm2);
  return hipGetLastError();
}

hipError_t launch_gemm2_big(const uint16_t* C, const uint8_t* w2, const float* s2,
                            const int32_t* counts, const int32_t* offsets, const float* sorted_w,
                            Gemm2Out dst, int H, int I, int E_l, int max_pairs, int rows_hint,
                            hipStream_t stream) {
  if (rows_hint < kB2TallRows) {
    const hipError_t e = launch_gemm2_big_t<kB2Ms, kB2ShortNs, kB2ShortD, kB2ShortWm, kB2ShortWn>(
        C, w2, s2, counts, offsets, sorted_w, dst, H, I, E_l, max_pairs, stream);
    if (e != hipErrorNotSupported) return e;  // I = 256: the 4-slot ring needs 3 K blocks
  }
  return launch_gemm2_big_t<kB2Ms, kB2Ns, kB2D, kB2Wm, kB2Wn>(C, w2, s2, counts, offsets,
                                                              sorted_w, dst, H, I, E_l,
                                                              max_pairs, stream);
}

}  // namespace jgmoe
