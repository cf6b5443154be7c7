// Activation quantisation: bf16 hidden states -> e4m3 codes with per-token 1x128 block scales,
// the producer of the operator's `hidden_states` / `hidden_states_scale` inputs.
//
// Rule (the reference applies it to its SwiGLU output before GEMM2,
// goal_full_shape/opus-4.8/moe_fp8_fwd/MOEDIR/main.py:151-156): per 128-column block of a row,
// amax = max |x|, scale = amax / 448 (0 for an all-zero block), codes = e4m3(clamp(x / s, -448,
// 448)) with s = scale, or 1 when scale is 0; fp32 arithmetic, correctly rounded division,
// round-to-nearest-even conversion. Scales are stored transposed, [H/128, T].
//
// Division. A correctly rounded fp32 division per element (about ten VALU instructions) costs
// more than the kernel's memory traffic, and the block's divisor s is shared by 128 elements.
// Each lane takes r = RN(1/s) once per block and corrects q0 = RN(x r) with one remainder step:
// q = RN(q0 + RN(x - q0 s) r), two FMAs (Markstein's division step; the remainder is exact
// while it does not underflow). copysign restores the sign of a zero x (the FMAs turn -0 into
// +0). Blocks with s < 2^-92, where a remainder could underflow for quotients that still matter,
// scale x and s by 2^100 first: exact, and the quotient is unchanged. On the GPU this gives the
// correctly rounded quotient's e4m3 code for every finite bf16 x with |x| <= amax under 4096
// block maxima (subnormal to largest finite), 1.35e8 pairs; the kernel's own test runs every
// finite bf16 value under 48 block maxima against the CPU oracle's division.
//
// HBM-bound (3 bytes per element plus 4 per 128 elements). A workgroup owns 16 (or 4) tokens x
// 512 columns: each wave quantises one token's 512 columns per pass (lane = 8 columns of one block;
// the block amax is a 16-lane xor reduction), so loads are 1 KiB and code stores 512 B per wave
// instruction; the workgroup's scales leave through LDS as four rows (one per block, 64 or 16
// bytes) of the transposed scale matrix.
#include "moe_device.h"
#include "moe_kernels.h"

namespace jgmoe {

namespace {

constexpr int kQBlk = 4;     // 128-column blocks per workgroup (512 columns)
// Tokens per workgroup. 16 (four per wave, one after another) for large batches; up to 1024
// tokens, 4 (one per wave), so a small batch spreads over four times the workgroups and each
// wave waits on one load instead of four. Kernel time per launch in a replayed graph (DS-V3
// H = 7168): T=16 3.8 -> 2.3 us, T=64 3.8 -> 2.4, T=256 4.0 -> 3.0, T=1024 6.0 -> 5.7; at
// T=16384 the 4-token form is slower (80 against 74 us). Loading a wave's four rows up front
// in the 16-token form took T=4096 from 16.1 to 17.5 us.
constexpr int kQTok = 16;
constexpr int kQTokSmall = 4;
constexpr int kQSmallT = 1024;
constexpr int kQWaves = 4;

// Four fp32 -> four e4m3 bytes (OCP e4m3fn on gfx950), round to nearest even. Inputs are
// already clamped to [-448, 448], so saturation never applies.
__device__ __forceinline__ uint32_t f32x4_to_e4m3(float a, float b, float c, float d) {
  int v = __builtin_amdgcn_cvt_pk_fp8_f32(a, b, 0, false);
  v = __builtin_amdgcn_cvt_pk_fp8_f32(c, d, v, true);
  return (uint32_t)v;
}

template <int TOK>
__global__ __launch_bounds__(kQWaves * kWave) void quant_act_kernel(
    const uint16_t* __restrict__ x, int T, int H, uint8_t* __restrict__ q,
    float* __restrict__ scale) {
  static_assert(TOK % kQWaves == 0 && kQBlk * TOK <= kWave, "one scale per lane of wave 0");
  __shared__ float sc[kQBlk][TOK];
  const int lane = threadIdx.x & (kWave - 1), w = wave_id();
  const int NB = H / kBlock;
  const int t0 = blockIdx.x * TOK, b0 = blockIdx.y * kQBlk;
  const int blk = b0 + (lane >> 4);  // this lane's 128-column block
  const bool active = blk < NB;
  const int col = blk * kBlock + 8 * (lane & 15);
  for (int j = w; j < TOK; j += kQWaves) {
    const int t = t0 + j;  // wave-uniform
    float v[8];
    float amax = 0.f;
    const bool live = t < T && active;  // uniform over each 16-lane block group
    if (live) {
      const uint4 raw = *(const uint4*)(x + (size_t)t * H + col);
      const uint32_t r[4] = {raw.x, raw.y, raw.z, raw.w};
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        v[2 * i] = __uint_as_float(r[i] << 16);
        v[2 * i + 1] = __uint_as_float(r[i] & 0xffff0000u);
      }
#pragma unroll
      for (int i = 0; i < 8; ++i) amax = fmaxf(amax, fabsf(v[i]));
    }
#pragma unroll
    for (int off = 8; off >= 1; off >>= 1) amax = fmaxf(amax, __shfl_xor(amax, off));
    const float cs = __fdiv_rn(amax, 448.0f);
    const float div = cs > 0.f ? cs : 1.0f;
    if (live) {
      const float up = div >= 0x1p-92f ? 1.0f : 0x1p100f;  // exact rescale of tiny blocks
      const float ds = div * up;
      const float rdiv = __fdiv_rn(1.0f, ds);
      float y[8];
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const float xs = v[i] * up;
        const float q0 = xs * rdiv;
        y[i] = copysignf(fmaf(fmaf(-q0, ds, xs), rdiv, q0), v[i]);
      }
#pragma unroll
      for (int i = 0; i < 8; ++i) y[i] = fminf(fmaxf(y[i], -448.0f), 448.0f);
      *(uint2*)(q + (size_t)t * H + col) =
          uint2{f32x4_to_e4m3(y[0], y[1], y[2], y[3]), f32x4_to_e4m3(y[4], y[5], y[6], y[7])};
    }
    if ((lane & 15) == 0) sc[lane >> 4][j] = cs;
  }
  __syncthreads();
  if (w == 0 && lane < kQBlk * TOK) {
    const int b = b0 + lane / TOK, t = t0 + lane % TOK;
    if (b < NB && t < T) scale[(size_t)b * T + t] = sc[lane / TOK][lane % TOK];
  }
}

}  // namespace

hipError_t launch_quantize_activations(const uint16_t* x, int T, int H, uint8_t* q, float* scale,
                                       hipStream_t stream) {
  const int NB = H / kBlock;
  if (T <= kQSmallT) {
    const dim3 grid((T + kQTokSmall - 1) / kQTokSmall, (NB + kQBlk - 1) / kQBlk);
    quant_act_kernel<kQTokSmall><<<grid, kQWaves * kWave, 0, stream>>>(x, T, H, q, scale);
    return hipGetLastError();
  }
  const dim3 grid((T + kQTok - 1) / kQTok, (NB + kQBlk - 1) / kQBlk);
  quant_act_kernel<kQTok><<<grid, kQWaves * kWave, 0, stream>>>(x, T, H, q, scale);
  return hipGetLastError();
}

}  // namespace jgmoe
