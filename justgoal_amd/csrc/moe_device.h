// Device-side helpers shared by the MoE kernels (gfx950 / CDNA4, wave64).
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace jgmoe {

constexpr int kBlock = 128;     // scale-block edge (1x128 activations, 128x128 weights)
constexpr int kWave = 64;
constexpr int kMaxTopK = 8;

typedef int v8i __attribute__((ext_vector_type(8)));
typedef float v4f __attribute__((ext_vector_type(4)));
typedef __bf16 v8bf __attribute__((ext_vector_type(8)));
typedef __bf16 v2bf __attribute__((ext_vector_type(2)));

// Wave index within the workgroup, as a wave-uniform (SGPR) value. Deriving it with a plain
// division leaves it in a VGPR as far as the compiler knows, and any buffer-load SGPR offset
// built from it then turns into a per-lane waterfall loop.
__device__ __forceinline__ int wave_id() {
  return __builtin_amdgcn_readfirstlane((int)(threadIdx.x / kWave));
}

// Marks a value the whole wave agrees on as uniform (SGPR). Needed where the compiler's
// divergence analysis loses track, e.g. values carried across loop iterations in structs.
__device__ __forceinline__ int uniform(int v) { return __builtin_amdgcn_readfirstlane(v); }
__device__ __forceinline__ uint32_t uniform(uint32_t v) {
  return (uint32_t)__builtin_amdgcn_readfirstlane((int)v);
}
template <class T>
__device__ __forceinline__ T* uniform(T* p) {
  const uint64_t v = (uint64_t)p;
  const uint32_t lo = uniform((uint32_t)v), hi = uniform((uint32_t)(v >> 32));
  return (T*)(((uint64_t)hi << 32) | lo);
}

__device__ __forceinline__ float bf16_bits_to_float(uint16_t b) {
  return __uint_as_float((uint32_t)b << 16);
}

// fp32 -> bf16 bits, round to nearest even (inputs here are finite).
__device__ __forceinline__ uint16_t float_to_bf16_bits(float f) {
  uint32_t u = __float_as_uint(f);
  u += 0x7fffu + ((u >> 16) & 1u);
  return (uint16_t)(u >> 16);
}

// Monotone map of a finite float onto uint32 (larger float -> larger key).
__device__ __forceinline__ uint32_t float_order_key(float v) {
  uint32_t u = __float_as_uint(v);
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

// Load of a T at a wave-uniform base plus a 32-bit per-lane byte offset (lets the compiler use
// the SGPR-base addressing form, one VGPR per address).
template <class T>
__device__ __forceinline__ T ldg(const void* base, uint32_t off) {
  return *(const T*)((const char*)base + off);
}

// Raw buffer resource over [base, base + bytes): loads take a per-lane 32-bit VGPR offset plus
// a wave-uniform SGPR offset, and anything past `bytes` reads as zero instead of faulting.
// 0x00020000 is the gfx9-family word-3 value for untyped raw access.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)bytes,
                                           0x00020000);
}

__device__ __forceinline__ uint4 buf_load16(__amdgpu_buffer_rsrc_t r, uint32_t voff,
                                            uint32_t soff) {
  typedef int v4i_ __attribute__((ext_vector_type(4)));
  const v4i_ v = __builtin_amdgcn_raw_buffer_load_b128(r, voff, soff, 0);
  return uint4{(uint32_t)v[0], (uint32_t)v[1], (uint32_t)v[2], (uint32_t)v[3]};
}

__device__ __forceinline__ uint32_t buf_load32b(__amdgpu_buffer_rsrc_t r, uint32_t voff,
                                                uint32_t soff) {
  return (uint32_t)__builtin_amdgcn_raw_buffer_load_b32(r, voff, soff, 0);
}

__device__ __forceinline__ v8i buf_load32(__amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t soff) {
  typedef int v4i_ __attribute__((ext_vector_type(4)));
  const v4i_ lo = __builtin_amdgcn_raw_buffer_load_b128(r, voff, soff, 0);
  const v4i_ hi = __builtin_amdgcn_raw_buffer_load_b128(r, voff + 16, soff, 0);
  return v8i{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
}

// ---- LDS DMA (buffer_load ... lds) -------------------------------------------------------------
// A DMA load moves 16 bytes per lane from global memory straight into LDS at
// lds_base + 16 * lane, bypassing VGPRs; the per-lane global offsets are free, so one
// instruction can fetch whole 128-byte lines while the LDS image gets any 16-byte permutation.
// The compiler counts these loads in vmcnt but cannot relate them to later LDS reads, so the
// kernels read DMA'd data with the asm reads below after an explicit vm_wait.
typedef __attribute__((address_space(3))) void* lds_ptr_t;

__device__ __forceinline__ void dma16(__amdgpu_buffer_rsrc_t r, void* lds_base, uint32_t voff,
                                      uint32_t soff) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (lds_ptr_t)lds_base, 16, voff, soff, 0, 0);
}

// 16-byte global load with the non-temporal hint, for data a kernel reads exactly once.
__device__ __forceinline__ uint4 load_nt16(const void* p) {
  typedef unsigned v4_t __attribute__((ext_vector_type(4)));
  const v4_t v = __builtin_nontemporal_load((const v4_t*)p);
  return uint4{v[0], v[1], v[2], v[3]};
}

// 16-byte global store with the non-temporal hint, for output nothing in the launch reads back.
__device__ __forceinline__ void store_nt16(void* p, uint4 v) {
  typedef unsigned v4_t __attribute__((ext_vector_type(4)));
  __builtin_nontemporal_store(v4_t{v.x, v.y, v.z, v.w}, (v4_t*)p);
}

// Cache-policy bit of gfx950 vector memory instructions marking a non-temporal (streaming)
// access.
constexpr int kCachePolicyNT = 2;

// dma16 for data this launch reads exactly once (the weight stream of the kernels that see each
// weight byte once per call): the non-temporal hint keeps those lines from displacing reused
// ones (activation rows, C fragments). Measured on the weight-streaming and LDS-tiled kernels,
// with three weight sets in rotation so no call finds its weights cached: DS-V3 T=64 call
// 146.9 -> 134.5 us, T=256 203.9 -> 188.6 us, Qwen3-style T=128 499.6 -> 474.4 us. The large-tile
// kernels, which reuse each weight tile across M-tiles through L2, got slower with it on every
// item (T=4096 GEMM1 217 -> 238 us); they use it only for experts with one M-tile (T=2048
// 311 -> 303 us, T=4096 448 -> 441 us, Qwen3-style T=1024 574 -> 556 us).
__device__ __forceinline__ void dma16_stream(__amdgpu_buffer_rsrc_t r, void* lds_base,
                                             uint32_t voff, uint32_t soff) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (lds_ptr_t)lds_base, 16, voff, soff, 0,
                                           kCachePolicyNT);
}

// 4 bytes per lane (e.g. one scale per row) into LDS at lds_base + 4 * lane.
__device__ __forceinline__ void dma4(__amdgpu_buffer_rsrc_t r, void* lds_base, uint32_t voff,
                                     uint32_t soff) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (lds_ptr_t)lds_base, 4, voff, soff, 0, 0);
}

// LDS byte address of a __shared__ object, as the 32-bit value DS instructions take.
__device__ __forceinline__ uint32_t lds_addr(const void* p) {
  return (uint32_t)(uintptr_t)(lds_ptr_t)p;
}

// Wait until at most N vector-memory operations of this wave are outstanding.
template <int N>
__device__ __forceinline__ void vm_wait() {
  static_assert(N >= 0 && N < 64, "vmcnt field is 6 bits");
  asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}

typedef uint32_t v4u __attribute__((ext_vector_type(4)));

__device__ __forceinline__ v4u ds_read16(uint32_t addr) {
  v4u v;
  asm volatile("ds_read_b128 %0, %1" : "=v"(v) : "v"(addr));
  return v;
}

__device__ __forceinline__ float ds_read4f(uint32_t addr) {
  float v;
  asm volatile("ds_read_b32 %0, %1" : "=v"(v) : "v"(addr));
  return v;
}

// Waits for every outstanding LDS read; follow with lds_fence on each value read by asm.
__device__ __forceinline__ void lds_wait_all() { asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory"); }
// Routes a value through an (ordered) asm after lds_wait_all, so no use of it can move above
// the wait.
__device__ __forceinline__ void lds_fence(v4u& x) { asm volatile("" : "+v"(x)); }
__device__ __forceinline__ void lds_fence(float& x) { asm volatile("" : "+v"(x)); }

// Completes the asm LDS reads that produced the arguments: the values flow through the wait,
// so no use of them can be scheduled before it.
__device__ __forceinline__ void lds_wait(v4u& x, v4u& y) {
  asm volatile("s_waitcnt lgkmcnt(0)" : "+v"(x), "+v"(y)::"memory");
}
__device__ __forceinline__ void lds_wait(v4u& x, v4u& y, v4u& z, v4u& w) {
  asm volatile("s_waitcnt lgkmcnt(0)" : "+v"(x), "+v"(y), "+v"(z), "+v"(w)::"memory");
}

// Weight K-block image in LDS: 16 rows x 128 bytes, row n's 16-byte chunk c stored at position
// c ^ wblk_swz(n). A DMA instruction h (h = 0, 1) fills rows 8h..8h+7 with whole lines; the MFMA
// operand read (lane = row n | group g, chunks 2g and 2g+1) is bank-conflict free.
// 16-byte chunk permutation of row n of a 16-row block (depends on n mod 16 only, so DMA code may
// pass a tile-level row). ds_read_b128 of the MFMA fragments (lane l reads row l&15, chunks
// 2(l>>4) and 2(l>>4)+1) measured conflict-free with (n & 7) ^ ((n >> 3) & 1) and 2-way
// conflicted with (n >> 1) & 7 or n & 7 (the hardware serves a b128 read in 16-lane groups).
__device__ __forceinline__ int wblk_swz(int row) {
  return (row & 7) ^ ((row >> 3) & 1);
}
// Global byte offset, relative to row 0 of the block, that lane `lane` of DMA instruction h
// fetches; `row_bytes` is the weight row pitch.
__device__ __forceinline__ uint32_t wblk_dma_off(int lane, int h, int row_bytes) {
  const int row = 8 * h + (lane >> 3);
  return (uint32_t)row * row_bytes + 16 * ((lane & 7) ^ wblk_swz(row));
}
// LDS offsets of the two 16-byte chunks lane (n = lane & 15, g = lane >> 4) reads.
__device__ __forceinline__ uint32_t wblk_read_off(int lane, int half) {
  const int n = lane & 15, g = lane >> 4;
  return n * 128 + 16 * ((2 * g + half) ^ wblk_swz(n));
}

// 16-byte chunk permutation of row n of a bf16 C tile in LDS (256-byte rows, one K block;
// depends on n mod 16). The fragment read (lane = row n | group g, chunks 4g..4g+3) took 21%
// less time with this permutation than with n & 15 in a ds_read_b128 probe.
__device__ __forceinline__ int crow_swz(int row) { return ((row & 7) << 1) | ((row >> 3) & 1); }

// Marks register values as used here, so the compiler completes their loads at this point (with
// a counted wait) instead of at a later overwrite of the same registers.
__device__ __forceinline__ void retire(float x) { asm volatile("" ::"v"(x)); }
__device__ __forceinline__ void retire(uint32_t x) { asm volatile("" ::"v"(x)); }
__device__ __forceinline__ void retire(int x) { asm volatile("" ::"v"(x)); }

// A row of up to 128 per-K-block scales held one per lane in two VGPRs. A K loop reads scale
// kb with a lane read (v_readlane) instead of a scalar memory load: scalar loads complete out of
// order and share their wait counter with LDS traffic, so consuming a prefetched one would wait
// for every outstanding scalar load and LDS access.
struct LaneScales {
  float v0, v1;
  __device__ __forceinline__ void load(const float* __restrict__ p, int n) {
    const int lane = threadIdx.x & (kWave - 1);
    v0 = lane < n ? p[lane] : 0.f;
    v1 = lane + kWave < n ? p[lane + kWave] : 0.f;
  }
  __device__ __forceinline__ float get(int kb) const {
    const float v = kb < kWave ? v0 : v1;
    return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), kb & (kWave - 1)));
  }
};

// One v_mfma_f32_16x16x128_f8f6f4 (both operands OCP e4m3), fresh accumulator.
// Operand layout (verified on gfx950): lane l supplies row/column (l & 15) and the 32 K-values
// [32*(l>>4), 32*(l>>4)+32) of the 128-wide K block; result lane l holds D[4*(l>>4)+i][l & 15].
__device__ __forceinline__ v4f mfma_f8_16x16x128(const v8i& a, const v8i& b) {
  v4f z = {0.f, 0.f, 0.f, 0.f};
  return __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(a, b, z, 0, 0, 0, 0, 0, 0);
}

// v_mfma_f32_16x16x32_bf16: lane l supplies row/column (l & 15), K-values [8*(l>>4), +8).
__device__ __forceinline__ v4f mfma_bf16_16x16x32(const v8bf& a, const v8bf& b, const v4f& c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}

// Four e4m3 bytes -> four bf16 (exact: every e4m3 value is representable in bf16).
__device__ __forceinline__ void fp8x4_to_bf16x4(int packed, v2bf& lo, v2bf& hi) {
  lo = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(packed, 1.0f, false);
  hi = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(packed, 1.0f, true);
}

// Maps a linear M-tile slot onto (local expert, first row within its segment) from the
// per-expert pair counts: each expert owns ceil(count / bm) consecutive slots. Every lane of
// the wave must call it; the result is wave-uniform. Returns false for slots past the end.
__device__ __forceinline__ bool find_m_tile(const int32_t* __restrict__ counts, int n_experts,
                                            int bm, int slot, int& expert, int& m0) {
  const int lane = threadIdx.x & (kWave - 1);
  int base = 0;
  for (int c0 = 0; c0 < n_experts; c0 += kWave) {
    const int ex = c0 + lane;
    const int n = ex < n_experts ? (counts[ex] + bm - 1) / bm : 0;
    int incl = n;
#pragma unroll
    for (int off = 1; off < kWave; off <<= 1) {
      int y = __shfl_up(incl, off);
      if (lane >= off) incl += y;
    }
    const int excl = incl - n;
    const bool hit = slot >= base + excl && slot < base + incl;
    const unsigned long long m = __ballot(hit);
    if (m) {
      const int src = __ffsll((long long)m) - 1;
      expert = c0 + src;
      m0 = (slot - base - __shfl(excl, src)) * bm;
      return true;
    }
    base += __shfl(incl, kWave - 1);
  }
  return false;
}

// Register-resident M-tile map for persistent kernels: lane l keeps expert l + 64*j (j < 4,
// so up to 256 local experts) with its pair count, segment offset and the inclusive prefix of
// tile counts. Built once per wave; each lookup is a ballot plus scalar lane reads.
struct TileMap {
  int incl[4], ntile[4], cnt[4], seg[4];
  int total;

  __device__ __forceinline__ void init(const int32_t* __restrict__ counts,
                                       const int32_t* __restrict__ offsets, int n_experts,
                                       int bm) {
    const int lane = threadIdx.x & (kWave - 1);
    int base = 0;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int ex = j * kWave + lane;
      const bool ok = ex < n_experts;
      cnt[j] = ok ? counts[ex] : 0;
      seg[j] = ok ? offsets[ex] : 0;
      ntile[j] = (cnt[j] + bm - 1) / bm;
      int x = ntile[j];
#pragma unroll
      for (int off = 1; off < kWave; off <<= 1) {
        const int y = __shfl_up(x, off);
        if (lane >= off) x += y;
      }
      incl[j] = base + x;
      base += __shfl(x, kWave - 1);
    }
    total = base;
  }

  // slot < total. Returns the local expert; m0 = first row of the tile within the segment.
  __device__ __forceinline__ int find(int slot, int bm, int& m0, int& count, int& segment) const {
    const int lane = threadIdx.x & (kWave - 1);
    int e = 0;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const unsigned long long m = __ballot(slot < incl[j] && slot >= incl[j] - ntile[j]);
      if (m) {
        const int src = __ffsll((long long)m) - 1;
        const int excl = __builtin_amdgcn_readlane(incl[j] - ntile[j], src);
        m0 = (slot - excl) * bm;
        count = __builtin_amdgcn_readlane(cnt[j], src);
        segment = __builtin_amdgcn_readlane(seg[j], src);
        e = j * kWave + src;
        break;
      }
    }
    (void)lane;
    return e;
  }
};

// The tile map of TileMap kept in LDS, for kernels whose register budget cannot hold the
// per-lane arrays for the whole kernel (a spilled copy would be reloaded from scratch, and every
// such reload waits for all outstanding vector-memory operations, LDS DMAs included).
constexpr int kMaxLocalExperts = 4 * kWave;
struct TileMapLds {
  int32_t incl[kMaxLocalExperts], cnt[kMaxLocalExperts], seg[kMaxLocalExperts];

  // Every wave calls this (all lanes); wave 0 stores the arrays. Returns the total tile count.
  // The caller must __syncthreads() before the first find().
  __device__ __forceinline__ int build(const int32_t* __restrict__ counts,
                                       const int32_t* __restrict__ offsets, int n_experts, int bm,
                                       bool store) {
    TileMap tm;
    tm.init(counts, offsets, n_experts, bm);
    if (store) {
      const int lane = threadIdx.x & (kWave - 1);
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        incl[j * kWave + lane] = tm.incl[j];
        cnt[j * kWave + lane] = tm.cnt[j];
        seg[j * kWave + lane] = tm.seg[j];
      }
    }
    return tm.total;
  }

  // Same contract as TileMap::find. Reads LDS with asm (lgkmcnt only).
  template <int BM>
  __device__ __forceinline__ int find(int slot, int n_experts, int& m0, int& count,
                                      int& segment) const {
    const int lane = threadIdx.x & (kWave - 1);
    const uint32_t bi = lds_addr(incl) + 4 * lane, bc = lds_addr(cnt) + 4 * lane,
                   bs = lds_addr(seg) + 4 * lane;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      if (j * kWave >= n_experts) break;
      float fi = ds_read4f(bi + 4 * kWave * j), fc = ds_read4f(bc + 4 * kWave * j),
            fs = ds_read4f(bs + 4 * kWave * j);
      lds_wait_all();
      lds_fence(fi);
      lds_fence(fc);
      lds_fence(fs);
      const int in = __float_as_int(fi), c = __float_as_int(fc);
      const int nt = (c + BM - 1) / BM;
      const unsigned long long m = __ballot(slot < in && slot >= in - nt);
      if (m) {
        const int src = __ffsll((long long)m) - 1;
        m0 = (slot - __builtin_amdgcn_readlane(in - nt, src)) * BM;
        count = __builtin_amdgcn_readlane(c, src);
        segment = __builtin_amdgcn_readlane(__float_as_int(fs), src);
        return j * kWave + src;
      }
    }
    return 0;
  }
};

// Total M-tiles over all experts: sum of ceil(count / bm). Wave-uniform; every lane must call.
__device__ __forceinline__ int count_m_tiles(const int32_t* __restrict__ counts, int n_experts,
                                             int bm) {
  const int lane = threadIdx.x & (kWave - 1);
  int n = 0;
  for (int ex = lane; ex < n_experts; ex += kWave) n += (counts[ex] + bm - 1) / bm;
#pragma unroll
  for (int off = kWave / 2; off >= 1; off >>= 1) n += __shfl_xor(n, off);
  return n;
}

}  // namespace jgmoe
