// Routing and token-permute kernels.
//
// route_kernel: one wave64 per token (4 tokens per workgroup up to T = 2048, 16 above), each
//   lane owning VPL = E/64 consecutive experts.
//   DeepSeek no-aux routing (reference semantics: goal_full_shape/fable-5.1/moe_fp8_fwd/MOEDIR/
//   moe_common.cuh:271-365, kda05_reproduction_single_shape/fable-5.1/moe_fp8_fwd/t14107/
//   moe_kernel.cu:482-600): sigmoid, + bias, group score = sum of the group's top two, keep
//   topk_group groups (ties -> lower group), top_k experts among kept groups (ties -> lower
//   expert), w = s / (sum s + 1e-20) * scaling. Softmax routing ranks by logit and renormalises.
//   Cross-lane steps are DPP row operations plus scalar lane reads (no LDS round trips): the
//   group top-2 merges inside the group's lanes, each top-k round is a DPP max of order keys
//   followed by a ballot that picks the lowest lane (= lowest expert index) holding it.
//   Each workgroup also writes its per-expert pair counts (one row of the chunk count table).
//
// permute_kernel: one workgroup per 64 tokens. From the count rows it derives the segment
//   offsets and this chunk's base inside each segment, then places its pairs: a pair's rank
//   inside its expert is a popcount over a per-expert token bitmask built with LDS atomic ORs
//   (order-independent). Tokens end up ascending inside each expert's segment (torch.nonzero
//   order) and the layout is identical from run to run; no global atomics, so the workspace
//   carries no state between calls.
#include "moe_device.h"
#include "moe_kernels.h"

namespace jgmoe {

namespace {

constexpr int kRouteWaves = 16;          // most tokens per routing workgroup (one wave each)
// Routing is VALU-latency-bound (sigmoid, DPP top-k chains): batches up to 2048 tokens use
// 4-token workgroups so their tokens spread over more CUs; larger ones keep 16 per workgroup so
// the permute kernel has fewer count rows to sum. Against a switch at 256 tokens, route +
// permute stage time: DS-V3 T=512 19.5 -> 16.8 us, T=1024 20.3 -> 17.6, T=2048 21.3 -> 20.1; at
// T=4096 the longer permute cancels the faster routing (22.9 against 24.1 us).
constexpr int kRouteSmallT = 2048, kRouteWavesSmall = 4;
__host__ __device__ __forceinline__ int route_tokens_per_group(int T) {
  return T <= kRouteSmallT ? kRouteWavesSmall : kRouteWaves;
}
constexpr int kPlaceTokens = 64;         // tokens per permute workgroup (one bitmask word)
constexpr int kMaxLocal = 256;           // local experts supported by the count / scan stages

template <int CTRL>
__device__ __forceinline__ uint32_t dpp(uint32_t x) {
  return (uint32_t)__builtin_amdgcn_update_dpp(0, (int)x, CTRL, 0xF, 0xF, false);
}

// Max over the wave: DPP reduction inside each row of 16 lanes, then four scalar lane reads.
__device__ __forceinline__ uint32_t wave_max_u32(uint32_t x) {
  x = max(x, dpp<0xB1>(x));   // quad_perm [1,0,3,2]
  x = max(x, dpp<0x4E>(x));   // quad_perm [2,3,0,1]
  x = max(x, dpp<0x141>(x));  // row_half_mirror
  x = max(x, dpp<0x140>(x));  // row_mirror
  const uint32_t a = __builtin_amdgcn_readlane(x, 0), b = __builtin_amdgcn_readlane(x, 16);
  const uint32_t c = __builtin_amdgcn_readlane(x, 32), d = __builtin_amdgcn_readlane(x, 48);
  return max(max(a, b), max(c, d));
}

// Value of the partner lane for a butterfly step of width `off` inside a group of lanes whose
// halves already hold uniform values (so a mirror pairs them as well as an xor would).
__device__ __forceinline__ float group_partner(float v, int off) {
  const uint32_t u = __float_as_uint(v);
  switch (off) {
    case 1: return __uint_as_float(dpp<0xB1>(u));
    case 2: return __uint_as_float(dpp<0x4E>(u));
    case 4: return __uint_as_float(dpp<0x141>(u));
    case 8: return __uint_as_float(dpp<0x140>(u));
    default: return __shfl_xor(v, off);
  }
}

// exp and sigmoid in fp32, step for step as the CPU oracle states them (oracle_sigmoid_f32):
// Cody-Waite range reduction (n = rint(y log2 e), r = y - n ln2 with a 16-bit ln2 head and its
// tail), e^r = 1 + r q(r) with q the degree-6 Taylor series of (e^r - 1) / r, and the rounding
// error of that last step kept as a low part; sigmoid = 1 / (1 + e^-x) with 1 + e^-x as a
// two-float sum and one Newton step on the correctly rounded reciprocal. Every product that
// feeds an add is an explicit fma, so contraction cannot change the bits. Within 1 ulp of the
// correctly rounded sigmoid.
__device__ __forceinline__ float exp_parts(float y, float& lo, int& n) {
  constexpr float kL2E = 1.44269504088896341f, kLn2Hi = 0.693145751953125f,
                  kLn2Lo = 1.428606765330187045e-06f;
  y = fminf(fmaxf(y, -104.0f), 88.0f);
  const float nf = rintf(y * kL2E);
  float r = __builtin_fmaf(-nf, kLn2Hi, y);
  r = __builtin_fmaf(-nf, kLn2Lo, r);
  float q = 1.0f / 5040.0f;
  q = __builtin_fmaf(q, r, 1.0f / 720.0f);
  q = __builtin_fmaf(q, r, 1.0f / 120.0f);
  q = __builtin_fmaf(q, r, 1.0f / 24.0f);
  q = __builtin_fmaf(q, r, 1.0f / 6.0f);
  q = __builtin_fmaf(q, r, 0.5f);
  q = __builtin_fmaf(q, r, 1.0f);
  const float h = __builtin_fmaf(r, q, 1.0f);
  lo = __builtin_fmaf(r, q, 1.0f - h);
  n = (int)nf;
  return h;
}

__device__ __forceinline__ float exp_f32(float y) {
  float lo;
  int n;
  const float h = exp_parts(y, lo, n);
  return ldexpf(h, n);
}

__device__ __forceinline__ float sigmoid_f32(float x) {
  const bool tiny = x < -87.0f;  // 1 + e^-x equals e^-x far below an ulp: the result is e^x
  float pl;
  int n;
  const float ph = exp_parts(tiny ? x : -x, pl, n);
  const float eh = ldexpf(ph, n), el = ldexpf(pl, n);
  const float dh = 1.0f + eh;
  const float dl = (eh >= 1.0f ? (eh - dh) + 1.0f : (1.0f - dh) + eh) + el;
  const float s0 = 1.0f / dh;
  const float res = __builtin_fmaf(-s0, dl, __builtin_fmaf(-s0, dh, 1.0f));
  return tiny ? eh : __builtin_fmaf(s0, res, s0);
}

__device__ __forceinline__ uint32_t order_key(float v) {
  return float_order_key(v + 0.0f);  // -0 -> +0 so that equal values tie on the index
}

// Routes one token (all 64 lanes active). Lanes k < top_k return selection k.
template <int VPL, int METHOD>
__device__ __forceinline__ void route_token(const float (&x)[VPL], const float (&bv)[VPL],
                                            int n_group, int topk_group, int top_k, float rsf,
                                            int& out_idx, float& out_w) {
  constexpr int E = VPL * kWave;
  const int lane = threadIdx.x & (kWave - 1);
  float s[VPL];
  uint32_t key[VPL];

  if (METHOD == ROUTING_DS) {
    float v[VPL];
#pragma unroll
    for (int j = 0; j < VPL; ++j) {
      s[j] = sigmoid_f32(x[j]);
      v[j] = s[j] + bv[j];
    }
    // top-2 (as a multiset) of this lane's values, then across the group's lanes
    float m1 = -INFINITY, m2 = -INFINITY;
#pragma unroll
    for (int j = 0; j < VPL; ++j) {
      if (v[j] > m1) {
        m2 = m1;
        m1 = v[j];
      } else if (v[j] > m2) {
        m2 = v[j];
      }
    }
    const int gsz = E / n_group;
    const int lpg = gsz / VPL;  // lanes per group, a power of two
    for (int off = 1; off < lpg; off <<= 1) {
      const float o1 = group_partner(m1, off), o2 = group_partner(m2, off);
      if (m1 >= o1) {
        m2 = fmaxf(m2, o1);
      } else {
        m2 = fmaxf(o2, m1);
        m1 = o1;
      }
    }
    const float gscore = gsz > 1 ? m1 + m2 : m1;
    const int g = lane / lpg;
    int rank = 0;
    for (int h = 0; h < n_group; ++h) {
      const float o = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(gscore), h * lpg));
      rank += (o > gscore) || (o == gscore && h < g);
    }
    const bool keep = rank < topk_group;
#pragma unroll
    for (int j = 0; j < VPL; ++j) key[j] = keep ? order_key(v[j]) : 0u;
  } else {
#pragma unroll
    for (int j = 0; j < VPL; ++j) {
      s[j] = x[j];
      key[j] = order_key(x[j]);
    }
  }

  int sel_idx[kMaxTopK];
  float sel_val[kMaxTopK];
#pragma unroll
  for (int k = 0; k < kMaxTopK; ++k) {
    sel_idx[k] = 0;
    sel_val[k] = 0.f;
    if (k < top_k) {
      // this lane's best remaining candidate (larger key, then lower index)
      uint32_t lb = key[0];
      int lj = 0;
#pragma unroll
      for (int j = 1; j < VPL; ++j)
        if (key[j] > lb) {
          lb = key[j];
          lj = j;
        }
      const uint32_t m = wave_max_u32(lb);
      const int src = __ffsll((long long)__ballot(lb == m)) - 1;  // lowest lane = lowest index
      const int jsel = __builtin_amdgcn_readlane(lj, src);
      float mine = s[0];
#pragma unroll
      for (int j = 1; j < VPL; ++j)
        if (lj == j) mine = s[j];
      sel_val[k] = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(mine), src));
      sel_idx[k] = src * VPL + jsel;
      if (lane == src) {
#pragma unroll
        for (int j = 0; j < VPL; ++j)
          if (j == jsel) key[j] = 0u;
      }
    }
  }

  // Lane k < top_k keeps selection k; the weights take the same operations per selection as the
  // definition, each lane evaluating only its own division (and, for softmax, its own exp).
  float mine = sel_val[0];
  int idx = sel_idx[0];
#pragma unroll
  for (int k = 1; k < kMaxTopK; ++k)
    if (lane == k) {
      mine = sel_val[k];
      idx = sel_idx[k];
    }
  out_idx = idx;
  if (METHOD == ROUTING_DS) {
    float sum = 0.0f;
#pragma unroll
    for (int k = 0; k < kMaxTopK; ++k)
      if (k < top_k) sum += sel_val[k];
    sum += 1e-20f;
    out_w = mine / sum * rsf;
  } else {
    const float ex = exp_f32(mine - sel_val[0]);
    float sum = 0.0f;
#pragma unroll
    for (int k = 0; k < kMaxTopK; ++k)
      if (k < top_k) sum += __int_as_float(__builtin_amdgcn_readlane(__float_as_int(ex), k));
    out_w = ex / sum;
  }
}


// (token, slot) -> local expert (or -1) and routing weight, for up to kPlaceTokens tokens.
struct TokenPairs {
  int le[kPlaceTokens][kMaxTopK];
  float w[kPlaceTokens][kMaxTopK];
};

__device__ __forceinline__ int local_of(int ge, int local_offset, int E_l) {
  const int le = ge - local_offset;
  return (le >= 0 && le < E_l) ? le : -1;
}

// Token membership per local expert: bit r of bits[e] is set when token row r selected e.
struct ExpertMasks {
  unsigned long long bits[kMaxLocal][kPlaceTokens / 64];
};

// Builds the masks of tp rows 0..n-1 (whole workgroup; LDS atomic ORs are order-independent)
// and cnt[e] = pairs of expert e among them. Ends with a barrier.
__device__ __forceinline__ void build_masks(const TokenPairs& tp, int n, int top_k, int E_l,
                                            ExpertMasks& m, int* cnt) {
  const int words = (n + 63) / 64;
  for (int i = threadIdx.x; i < E_l * words; i += blockDim.x) m.bits[i / words][i % words] = 0ull;
  __syncthreads();
  for (int i = threadIdx.x; i < n * top_k; i += blockDim.x) {
    const int r = i / top_k, k = i % top_k;
    const int e = tp.le[r][k];
    if (e >= 0) atomicOr(&m.bits[e][r >> 6], 1ull << (r & 63));
  }
  __syncthreads();
  for (int e = threadIdx.x; e < E_l; e += blockDim.x) {
    int c = 0;
    for (int w = 0; w < words; ++w) c += __popcll(m.bits[e][w]);
    cnt[e] = c;
  }
  __syncthreads();
}

// Places tp rows 0..n-1 (tokens t0..t0+n-1): pair (r, k) of expert e goes to base[e] plus the
// number of earlier rows that also selected e, so each segment stays in ascending token order.
__device__ __forceinline__ void place_from_masks(const TokenPairs& tp, const ExpertMasks& m,
                                                 int n, int t0, int T, int top_k,
                                                 const int* base, int k_local,
                                                 int32_t* __restrict__ sorted_tok,
                                                 float* __restrict__ sorted_w,
                                                 int32_t* __restrict__ pair_dst,
                                                 int32_t* __restrict__ pair_of) {
  for (int i = threadIdx.x; i < n * top_k; i += blockDim.x) {
    const int r = i / top_k, k = i % top_k, t = t0 + r;
    const int e = tp.le[r][k];
    if (e >= 0) {
      int rank = __popcll(m.bits[e][r >> 6] & ((1ull << (r & 63)) - 1ull));
      for (int w = 0; w < (r >> 6); ++w) rank += __popcll(m.bits[e][w]);
      const int p = base[e] + rank;
      // Rank of this pair among the token's local pairs in ascending local-expert order: the
      // first goes straight into the output row, the others into the token's partial rows.
      int j = 0;
#pragma unroll
      for (int q = 0; q < kMaxTopK; ++q) {
        const int o = tp.le[r][q];
        j += (o >= 0 && o < e);
      }
      sorted_tok[p] = t;
      sorted_w[p] = tp.w[r][k];
      pair_dst[p] = j == 0 ? t : -(1 + t * (k_local - 1) + (j - 1));
      pair_of[(size_t)t * top_k + k] = p;
    } else if (t < T) {
      pair_of[(size_t)t * top_k + k] = -1;
    }
  }
}

// Exclusive prefix over n <= 256 ints by one wave (4 per lane) into out[0..n].
__device__ __forceinline__ void wave_exclusive_scan(const int* in, int* out, int n) {
  const int lane = threadIdx.x & (kWave - 1);
  int v[4], tot = 0;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int e = lane * 4 + j;
    v[j] = e < n ? in[e] : 0;
    tot += v[j];
  }
  int incl = tot;
#pragma unroll
  for (int off = 1; off < kWave; off <<= 1) {
    const int y = __shfl_up(incl, off);
    if (lane >= off) incl += y;
  }
  int run = incl - tot;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int e = lane * 4 + j;
    if (e < n) out[e] = run;
    run += v[j];
  }
  if (lane == kWave - 1) out[n] = incl;
}

}  // namespace

template <int VPL, int METHOD>
__global__ __launch_bounds__(1024) void route_kernel(
    const float* __restrict__ logits, const uint16_t* __restrict__ bias, int T, int n_group,
    int topk_group, int top_k, float rsf, int local_offset, int E_l, int32_t* __restrict__ topk_idx,
    float* __restrict__ topk_w, int32_t* __restrict__ hist) {
  constexpr int E = VPL * kWave;
  __shared__ TokenPairs tp;  // rows 0..tpw-1 used
  __shared__ ExpertMasks masks;
  __shared__ int cnt[kMaxLocal];
  const int lane = threadIdx.x & (kWave - 1), wave = wave_id();
  const int tpw = blockDim.x / kWave;  // tokens of this workgroup
  const int t0 = blockIdx.x * tpw;
  const int t = t0 + wave;

  int le = -1;
  float w = 0.f;
  if (t < T) {  // wave-uniform
    float bv[VPL], x[VPL];
#pragma unroll
    for (int j = 0; j < VPL; ++j) {
      x[j] = logits[(size_t)t * E + lane * VPL + j];
      bv[j] = (METHOD == ROUTING_DS && bias) ? bf16_bits_to_float(bias[lane * VPL + j]) : 0.0f;
    }
    int idx;
    route_token<VPL, METHOD>(x, bv, n_group, topk_group, top_k, rsf, idx, w);
    if (lane < top_k) {
      topk_idx[(size_t)t * top_k + lane] = idx;
      topk_w[(size_t)t * top_k + lane] = w;
      le = local_of(idx, local_offset, E_l);
    }
  }
  if (lane < kMaxTopK) {
    tp.le[wave][lane] = le;
    tp.w[wave][lane] = w;
  }
  __syncthreads();
  build_masks(tp, tpw, top_k, E_l, masks, cnt);
  for (int e = threadIdx.x; e < E_l; e += blockDim.x) hist[(size_t)blockIdx.x * E_l + e] = cnt[e];
}

__global__ __launch_bounds__(256) void permute_kernel(
    const int32_t* __restrict__ topk_idx, const float* __restrict__ topk_w,
    const int32_t* __restrict__ hist, int T, int K, int local_offset, int E_l, int n_rows,
    int32_t* __restrict__ counts, int32_t* __restrict__ offsets,
    int32_t* __restrict__ sorted_tok, float* __restrict__ sorted_w,
    int32_t* __restrict__ pair_dst, int32_t* __restrict__ pair_of) {
  __shared__ TokenPairs tp;  // rows 0..63 used
  __shared__ ExpertMasks masks;
  __shared__ int chunk_cnt[kMaxLocal];
  __shared__ int total[kMaxLocal];
  __shared__ int before[kMaxLocal];
  __shared__ int off[kMaxLocal + 1];
  const int t0 = blockIdx.x * kPlaceTokens;
  const int row0 = t0 / route_tokens_per_group(T);  // first count row of this chunk
  // Column sums of the count table. For tables of 64 rows or more (T > 256) and E_l a multiple
  // of 4, thread (q, slice) adds columns 4q..4q+3 of every n_slices-th row with 16-byte loads,
  // sixteen rows in flight (T = 16384: 32 rows per thread instead of 128; permute 27.8 -> 12.8 us,
  // T = 4096 13.9 -> 11.2 us); otherwise thread (e, slice) adds column e, eight rows in flight.
  const bool quads = (E_l & 3) == 0 && n_rows >= 64;
  const int cols = quads ? E_l / 4 : E_l;
  const int n_slices = max(1, (int)blockDim.x / cols);
  const int e = threadIdx.x % cols, slice = threadIdx.x / cols;
  if (threadIdx.x < E_l) {
    total[threadIdx.x] = 0;
    before[threadIdx.x] = 0;
  }
  __syncthreads();
  if (quads && slice < n_slices) {
    int4 a = {0, 0, 0, 0}, b = {0, 0, 0, 0};
    for (int r0 = slice; r0 < n_rows; r0 += 16 * n_slices) {
      int4 h[16];
#pragma unroll
      for (int u = 0; u < 16; ++u) {
        const int r = r0 + u * n_slices;
        h[u] = r < n_rows ? *(const int4*)(hist + (size_t)r * E_l + 4 * e) : int4{0, 0, 0, 0};
      }
#pragma unroll
      for (int u = 0; u < 16; ++u) {
        const bool bf = (r0 + u * n_slices) < row0;
        a.x += h[u].x;
        a.y += h[u].y;
        a.z += h[u].z;
        a.w += h[u].w;
        b.x += bf ? h[u].x : 0;
        b.y += bf ? h[u].y : 0;
        b.z += bf ? h[u].z : 0;
        b.w += bf ? h[u].w : 0;
      }
    }
    atomicAdd(&total[4 * e], a.x);
    atomicAdd(&total[4 * e + 1], a.y);
    atomicAdd(&total[4 * e + 2], a.z);
    atomicAdd(&total[4 * e + 3], a.w);
    atomicAdd(&before[4 * e], b.x);
    atomicAdd(&before[4 * e + 1], b.y);
    atomicAdd(&before[4 * e + 2], b.z);
    atomicAdd(&before[4 * e + 3], b.w);
  } else if (!quads && slice < n_slices) {
    int a = 0, b = 0;
    for (int r0 = slice; r0 < n_rows; r0 += 8 * n_slices) {
      int h[8];
#pragma unroll
      for (int u = 0; u < 8; ++u) {
        const int r = r0 + u * n_slices;
        h[u] = r < n_rows ? hist[(size_t)r * E_l + e] : 0;
      }
#pragma unroll
      for (int u = 0; u < 8; ++u) {
        a += h[u];
        b += (r0 + u * n_slices) < row0 ? h[u] : 0;
      }
    }
    atomicAdd(&total[e], a);
    atomicAdd(&before[e], b);
  }
  for (int i = threadIdx.x; i < kPlaceTokens * kMaxTopK; i += blockDim.x) {
    const int r = i / kMaxTopK, k = i % kMaxTopK, t = t0 + r;
    int l = -1;
    float w = 0.f;
    if (t < T && k < K) {
      l = local_of(topk_idx[(size_t)t * K + k], local_offset, E_l);
      w = topk_w[(size_t)t * K + k];
    }
    tp.le[r][k] = l;
    tp.w[r][k] = w;
  }
  __syncthreads();
  const int n = min(kPlaceTokens, T - t0);
  build_masks(tp, n, K, E_l, masks, chunk_cnt);
  if (wave_id() == 0) wave_exclusive_scan(total, off, E_l);
  __syncthreads();
  if (blockIdx.x == 0)
    for (int i = threadIdx.x; i <= E_l; i += blockDim.x) {
      offsets[i] = off[i];
      if (i < E_l) counts[i] = total[i];
    }
  if (threadIdx.x < E_l) before[threadIdx.x] += off[threadIdx.x];
  __syncthreads();
  place_from_masks(tp, masks, n, t0, T, K, before, min(K, E_l), sorted_tok, sorted_w, pair_dst,
                   pair_of);
}

int route_chunks(int T) {
  const int tpw = route_tokens_per_group(T);
  return (T + tpw - 1) / tpw;
}

hipError_t launch_route(const float* logits, const uint16_t* bias, int T, int E, int n_group,
                        int topk_group, int top_k, int method, float rsf, int local_offset,
                        int E_l, int32_t* topk_idx, float* topk_w, int32_t* hist,
                        hipStream_t stream) {
  if (E_l > kMaxLocal || top_k > kMaxTopK) return hipErrorInvalidValue;
  const dim3 grid(route_chunks(T)), block(route_tokens_per_group(T) * kWave);
#define JG_ROUTE(VPL)                                                                        \
  if (E == VPL * kWave) {                                                                    \
    if (method == ROUTING_DS)                                                                \
      route_kernel<VPL, ROUTING_DS><<<grid, block, 0, stream>>>(                             \
          logits, bias, T, n_group, topk_group, top_k, rsf, local_offset, E_l, topk_idx,     \
          topk_w, hist);                                                                     \
    else                                                                                     \
      route_kernel<VPL, ROUTING_SOFTMAX><<<grid, block, 0, stream>>>(                        \
          logits, bias, T, n_group, topk_group, top_k, rsf, local_offset, E_l, topk_idx,     \
          topk_w, hist);                                                                     \
    return hipGetLastError();                                                                \
  }
  JG_ROUTE(1)
  JG_ROUTE(2)
  JG_ROUTE(4)
  JG_ROUTE(8)
#undef JG_ROUTE
  return hipErrorInvalidValue;
}

hipError_t launch_permute(const int32_t* topk_idx, const float* topk_w, const int32_t* hist,
                          int T, int K, int local_offset, int E_l, int32_t* counts,
                          int32_t* offsets, int32_t* sorted_tok, float* sorted_w,
                          int32_t* pair_dst, int32_t* pair_of, hipStream_t stream) {
  const int blocks = (T + kPlaceTokens - 1) / kPlaceTokens;
  permute_kernel<<<dim3(blocks), dim3(256), 0, stream>>>(topk_idx, topk_w, hist, T, K,
                                                        local_offset, E_l, route_chunks(T),
                                                        counts, offsets, sorted_tok, sorted_w,
                                                        pair_dst, pair_of);
  return hipGetLastError();
}

}  // namespace jgmoe
