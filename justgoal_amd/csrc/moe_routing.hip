// Routing and token-permute kernels.
//
// route_kernel: one wave64 per token, each lane owns VPL = E/64 consecutive experts.
//   DeepSeek no-aux routing (reference semantics: goal_full_shape/fable-5.1/moe_fp8_fwd/MOEDIR/
//   moe_common.cuh:271-365, kda05_reproduction_single_shape/fable-5.1/moe_fp8_fwd/t14107/
//   moe_kernel.cu:482-600): sigmoid, + bias, group score = sum of the group's top two, keep
//   topk_group groups (ties -> lower group), top_k experts among kept groups (ties -> lower
//   expert), w = s / (sum s + 1e-20) * scaling. Softmax routing ranks by logit and renormalises.
//   Everything stays in registers: group reductions are xor-shuffles inside the group's lanes and
//   each top-k round is a 64-bit (order key, ~index) wave max.
//
// permute_kernel: one workgroup per local expert, a deterministic stable compaction of the
//   tokens that selected it (ascending token order = torch.nonzero order). No atomics, so the
//   workspace needs no zeroing and the layout is identical from run to run.
#include "moe_device.h"
#include "moe_kernels.h"

namespace jgmoe {

__device__ __forceinline__ unsigned long long make_key(float v, int idx) {
  v = v + 0.0f;  // -0 -> +0 so that equal values tie on the index
  return ((unsigned long long)float_order_key(v) << 32) | (uint32_t)(~(uint32_t)idx);
}

template <int VPL, int METHOD>
__global__ __launch_bounds__(256) void route_kernel(const float* __restrict__ logits,
                                                    const uint16_t* __restrict__ bias, int T,
                                                    int n_group, int topk_group, int top_k,
                                                    float rsf, int32_t* __restrict__ topk_idx,
                                                    float* __restrict__ topk_w) {
  constexpr int E = VPL * kWave;
  const int lane = threadIdx.x & (kWave - 1);
  const int t = blockIdx.x * (blockDim.x / kWave) + wave_id();
  if (t >= T) return;  // wave-uniform

  float x[VPL];
  const float* xr = logits + (size_t)t * E + lane * VPL;
#pragma unroll
  for (int j = 0; j < VPL; ++j) x[j] = xr[j];

  float s[VPL];
  unsigned long long key[VPL];
  if (METHOD == ROUTING_DS) {
    float v[VPL];
#pragma unroll
    for (int j = 0; j < VPL; ++j) {
      s[j] = (float)(1.0 / (1.0 + exp(-(double)x[j])));
      v[j] = s[j] + (bias ? bf16_bits_to_float(bias[lane * VPL + j]) : 0.0f);
    }
    // top-2 (as a multiset) of this lane's values, then of the group's lanes
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
    const int lpg = (E / n_group) / VPL;  // lanes per group, a power of two
    for (int off = 1; off < lpg; off <<= 1) {
      const float o1 = __shfl_xor(m1, off), o2 = __shfl_xor(m2, off);
      if (m1 >= o1) {
        m2 = fmaxf(m2, o1);
      } else {
        m2 = fmaxf(o2, m1);
        m1 = o1;
      }
    }
    const float gscore = (E / n_group > 1) ? m1 + m2 : m1;
    const int g = lane / lpg;
    int rank = 0;
    for (int h = 0; h < n_group; ++h) {
      const float o = __shfl(gscore, h * lpg);
      rank += (o > gscore) || (o == gscore && h < g);
    }
    const bool keep = rank < topk_group;
#pragma unroll
    for (int j = 0; j < VPL; ++j) key[j] = keep ? make_key(v[j], lane * VPL + j) : 0ull;
  } else {
#pragma unroll
    for (int j = 0; j < VPL; ++j) {
      s[j] = x[j];
      key[j] = make_key(x[j], lane * VPL + j);
    }
  }

  int sel_idx[kMaxTopK];
  float sel_val[kMaxTopK];
#pragma unroll
  for (int k = 0; k < kMaxTopK; ++k) {
    sel_idx[k] = 0;
    sel_val[k] = 0.f;
    if (k < top_k) {
      unsigned long long best = key[0];
#pragma unroll
      for (int j = 1; j < VPL; ++j) best = key[j] > best ? key[j] : best;
#pragma unroll
      for (int off = kWave / 2; off >= 1; off >>= 1) {
        const unsigned long long o = __shfl_xor(best, off);
        best = o > best ? o : best;
      }
      const int idx = (int)(~(uint32_t)best);
      float mine = s[0];
#pragma unroll
      for (int j = 0; j < VPL; ++j) {
        if (lane * VPL + j == idx) key[j] = 0ull;
        if ((idx % VPL) == j) mine = s[j];
      }
      sel_idx[k] = idx;
      sel_val[k] = __shfl(mine, idx / VPL);
    }
  }

  float w[kMaxTopK];
  if (METHOD == ROUTING_DS) {
    float sum = 0.0f;
#pragma unroll
    for (int k = 0; k < kMaxTopK; ++k)
      if (k < top_k) sum += sel_val[k];
    sum += 1e-20f;
#pragma unroll
    for (int k = 0; k < kMaxTopK; ++k) w[k] = sel_val[k] / sum * rsf;
  } else {
    float ex[kMaxTopK];
    float sum = 0.0f;
#pragma unroll
    for (int k = 0; k < kMaxTopK; ++k) {
      ex[k] = (float)exp((double)(sel_val[k] - sel_val[0]));
      if (k < top_k) sum += ex[k];
    }
#pragma unroll
    for (int k = 0; k < kMaxTopK; ++k) w[k] = ex[k] / sum;
  }
  if (lane < top_k) {
    int oi = sel_idx[0];
    float ow = w[0];
#pragma unroll
    for (int k = 1; k < kMaxTopK; ++k)
      if (lane == k) {
        oi = sel_idx[k];
        ow = w[k];
      }
    topk_idx[(size_t)t * top_k + lane] = oi;
    topk_w[(size_t)t * top_k + lane] = ow;
  }
}

// Block-wide sum over 256 threads (4 waves).
__device__ __forceinline__ int block_sum_256(int v, int* red) {
#pragma unroll
  for (int off = kWave / 2; off >= 1; off >>= 1) v += __shfl_xor(v, off);
  const int wave = threadIdx.x / kWave;
  __syncthreads();
  if ((threadIdx.x & (kWave - 1)) == 0) red[wave] = v;
  __syncthreads();
  return red[0] + red[1] + red[2] + red[3];
}

__global__ __launch_bounds__(256) void permute_kernel(const int32_t* __restrict__ topk_idx,
                                                      const float* __restrict__ topk_w, int T,
                                                      int K, int local_offset, int E_l,
                                                      int32_t* __restrict__ counts,
                                                      int32_t* __restrict__ offsets,
                                                      int32_t* __restrict__ sorted_tok,
                                                      float* __restrict__ sorted_w,
                                                      int32_t* __restrict__ pair_of) {
  __shared__ int red[4];
  __shared__ int wcnt[4];
  const int e = blockIdx.x;
  const int tid = threadIdx.x;
  const int lane = tid & (kWave - 1), wave = tid / kWave;

  // pass 1: pairs of lower local experts (= this segment's offset) and of this expert
  int lt = 0, eq = 0;
  for (int t = tid; t < T; t += 256) {
    for (int k = 0; k < K; ++k) {
      const int le = topk_idx[(size_t)t * K + k] - local_offset;
      lt += (le >= 0 && le < e);
      eq += (le == e);
    }
  }
  const int base = block_sum_256(lt, red);
  const int cnt = block_sum_256(eq, red);
  if (tid == 0) {
    counts[e] = cnt;
    offsets[e] = base;
    if (e == E_l - 1) offsets[E_l] = base + cnt;
  }

  // pass 2: stable placement, 256 tokens per step
  int running = 0;
  for (int t0 = 0; t0 < T; t0 += 256) {
    const int t = t0 + tid;
    int slot = -1;
    if (t < T) {
      for (int k = 0; k < K; ++k) {
        const int le = topk_idx[(size_t)t * K + k] - local_offset;
        if (le == e) slot = k;
        if (e == 0 && (le < 0 || le >= E_l)) pair_of[(size_t)t * K + k] = -1;
      }
    }
    const unsigned long long m = __ballot(slot >= 0);
    const int pre = __popcll(m & ((1ull << lane) - 1ull));
    __syncthreads();
    if (lane == 0) wcnt[wave] = __popcll(m);
    __syncthreads();
    int woff = 0;
    for (int w = 0; w < wave; ++w) woff += wcnt[w];
    const int total = wcnt[0] + wcnt[1] + wcnt[2] + wcnt[3];
    if (slot >= 0) {
      const int p = base + running + woff + pre;
      sorted_tok[p] = t;
      sorted_w[p] = topk_w[(size_t)t * K + slot];
      pair_of[(size_t)t * K + slot] = p;
    }
    running += total;
  }
}

hipError_t launch_route(const float* logits, const uint16_t* bias, int T, int E, int n_group,
                        int topk_group, int top_k, int method, float rsf, int32_t* topk_idx,
                        float* topk_w, hipStream_t stream) {
  const dim3 grid((T + 3) / 4), block(256);
#define JG_ROUTE(VPL)                                                                        \
  if (E == VPL * kWave) {                                                                    \
    if (method == ROUTING_DS)                                                                \
      route_kernel<VPL, ROUTING_DS><<<grid, block, 0, stream>>>(                             \
          logits, bias, T, n_group, topk_group, top_k, rsf, topk_idx, topk_w);               \
    else                                                                                     \
      route_kernel<VPL, ROUTING_SOFTMAX><<<grid, block, 0, stream>>>(                        \
          logits, bias, T, n_group, topk_group, top_k, rsf, topk_idx, topk_w);               \
    return hipGetLastError();                                                                \
  }
  JG_ROUTE(1)
  JG_ROUTE(2)
  JG_ROUTE(4)
  JG_ROUTE(8)
#undef JG_ROUTE
  return hipErrorInvalidValue;
}

hipError_t launch_permute(const int32_t* topk_idx, const float* topk_w, int T, int K,
                          int local_offset, int E_l, int32_t* counts, int32_t* offsets,
                          int32_t* sorted_tok, float* sorted_w, int32_t* pair_of,
                          hipStream_t stream) {
  permute_kernel<<<dim3(E_l), dim3(256), 0, stream>>>(topk_idx, topk_w, T, K, local_offset, E_l,
                                                      counts, offsets, sorted_tok, sorted_w,
                                                      pair_of);
  return hipGetLastError();
}

}  // namespace jgmoe
