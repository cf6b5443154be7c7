/*
 * justgoal_moe.h -- C ABI of the MI355X (gfx950) FP8 block-scale Mixture-of-Experts operator.
 *
 * Drop-in boundary for the reference solutions' C entry points. Every pointer is a device
 * pointer; every buffer is owned by the caller. Calls enqueue work on `stream` (a hipStream_t,
 * NULL = the default stream) and return without synchronising the host. They never throw and
 * never allocate device memory.
 *
 * Return codes: 0 on success; MOE_ERR_* (negative) for argument or geometry errors detected on
 * the host before anything is enqueued; otherwise a positive hipError_t from a launch.
 *
 * Layouts (row-major, contiguous; T tokens, H hidden, I intermediate, E global experts,
 * E_l local experts, B = 128):
 *   logits      fp32        [T, E]
 *   bias        bf16        [E]            (may be NULL: treated as zeros)
 *   hs          fp8 e4m3fn  [T, H]
 *   hs_scale    fp32        [H/B, T]       per-token 1x128 block scales, transposed
 *   w13         fp8 e4m3fn  [E_l, 2I, H]   rows 0..I-1 = X1 (linear half), I..2I-1 = X2 (gated half)
 *   s13         fp32        [E_l, 2I/B, H/B]
 *   w2          fp8 e4m3fn  [E_l, H, I]
 *   s2          fp32        [E_l, H/B, I/B]
 *   out         bf16        [T, H]
 */
#ifndef JUSTGOAL_MOE_H
#define JUSTGOAL_MOE_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define MOE_OK 0
#define MOE_ERR_INVALID_ARG (-1)     /* null pointer, negative T, T above the limit, bad scalar */
#define MOE_ERR_GEOMETRY (-2)        /* geometry the kernels do not support */
#define MOE_ERR_NO_DEVICE (-3)       /* device query failed or the device is not gfx950 */
#define MOE_ERR_SCRATCH_SIZE (-4)    /* moe_run_noalloc: the call needs more than its scratch */

#define MOE_ROUTING_DS 0             /* sigmoid + bias, group-limited top-k, renorm x scaling */
#define MOE_ROUTING_SOFTMAX 1        /* softmax top-k, renormalised */

/* Operator geometry. The DeepSeek-V3 values are {7168, 2048, 256, 32, 8, 8, 4, MOE_ROUTING_DS}. */
typedef struct moe_geometry {
  int hidden;          /* H, multiple of 128, at most 16384 */
  int intermediate;    /* I, multiple of 128, at most 16384 */
  int num_experts;     /* E, multiple of 64, <= 512 */
  int local_experts;   /* E_l, 1..min(E, 256) */
  int top_k;           /* 1..8 */
  int n_group;         /* groups for MOE_ROUTING_DS (1 for softmax) */
  int topk_group;      /* groups kept per token */
  int routing_method;  /* MOE_ROUTING_* */
} moe_geometry;

/*
 * DeepSeek-V3 operator, fixed geometry.
 * Replaces: `extern "C" int moe_run(...)`
 *   kda05_reproduction_single_shape/fable-5.1/moe_fp8_fwd/t1/kernel.cu:743-790
 * and the value-returning Python entry `run(...)` it backs
 *   goal_full_shape/opus-4.8/moe_fp8_fwd/MOEDIR/main.py:286-288.
 * Same argument order and meaning. Difference: the workspace need not be zeroed on entry (the
 * reference requires a zeroed one, t1/main.py:77-83; no kernel here keeps state in it), and it
 * is sized by moe_workspace_bytes(T). Calls that overlap in time need distinct workspaces.
 * T is limited by 32-bit buffer offsets: T*hidden < 2^31 - 16 and T*min(top_k, E_local)*
 * intermediate*2 < 2^31 (DS-V3: T <= 65535); larger T returns MOE_ERR_INVALID_ARG.
 */
int moe_run(const void* logits, const void* bias, const void* hs, const void* hs_scale,
            const void* w13, const void* s13, const void* w2, const void* s2, int local_offset,
            float scaling, void* out, void* workspace, int T, void* stream);

/*
 * Workspace bytes moe_run needs for T tokens.
 * Replaces: `extern "C" int moe_workspace_bytes(int T)` (t1/kernel.cu:741), same signature (the
 * reference binds it with restype c_int, t1/main.py:64-65). DS-V3 needs about 133 KiB per
 * token (bf16 C rows and bf16 partial rows): 1.88 GB at T = 14107. A size that does not fit in
 * an int (T above 16107) returns MOE_ERR_INVALID_ARG; moe_workspace_bytes_ex gives it as int64.
 */
int moe_workspace_bytes(int T);

/* moe_run for any supported geometry (the reference hard-codes DS-V3; same arguments otherwise). */
int moe_run_ex(const moe_geometry* geom, const void* logits, const void* bias, const void* hs,
               const void* hs_scale, const void* w13, const void* s13, const void* w2,
               const void* s2, int local_offset, float scaling, void* out, void* workspace, int T,
               void* stream);

/* Workspace bytes for moe_run_ex; -MOE_ERR_* style negative value on a bad geometry. */
int64_t moe_workspace_bytes_ex(const moe_geometry* geom, int T);

/*
 * moe_run_ex without a workspace argument, for callers that cannot allocate device memory
 * (code under HIP graph capture, tight serving loops, harnesses that forbid hipMalloc). No
 * counterpart in the reference. It calls no allocator: the workspace is a fixed array of
 * MOE_NOALLOC_SCRATCH_BYTES in the library's device code, one per GPU, held until the process
 * ends (its device address is looked up once per device on the first call there). A call whose
 * moe_workspace_bytes_ex exceeds that size returns MOE_ERR_SCRATCH_SIZE before enqueueing
 * anything (DS-V3: up to 503 tokens; the Qwen3-style geometry: up to 815). Every call on a GPU
 * shares that GPU's array: calls that overlap in time on one GPU (other streams, other host
 * threads) race and must not be issued; calls ordered on one stream are fine.
 */
#define MOE_NOALLOC_SCRATCH_BYTES (64u << 20)
int moe_run_noalloc(const moe_geometry* geom, const void* logits, const void* bias,
                    const void* hs, const void* hs_scale, const void* w13, const void* s13,
                    const void* w2, const void* s2, int local_offset, float scaling, void* out,
                    int T, void* stream);

/*
 * Routing + permute stages only (the first two kernels of moe_run_ex), leaving their outputs in
 * the workspace regions described by moe_workspace_layout. The reference has these as the
 * first kernels of its pipeline (goal_full_shape/opus-4.8/moe_fp8_fwd/MOEDIR/main.py:244-248);
 * exported so their integer outputs can be checked bit-exactly.
 */
int moe_route_ex(const moe_geometry* geom, const void* logits, const void* bias, int local_offset,
                 float scaling, void* workspace, int T, void* stream);

/* Workspace regions, in order; moe_workspace_layout writes their byte offsets. */
enum {
  MOE_WS_TOPK_IDX = 0,   /* int32 [T, top_k]  global expert ids in selection order */
  MOE_WS_TOPK_W,         /* fp32  [T, top_k]  routing weights */
  MOE_WS_PAIR_OF,        /* int32 [T, top_k]  pair row of slot (t,k), -1 if not local */
  MOE_WS_COUNTS,         /* int32 [E_l]       pairs per local expert */
  MOE_WS_OFFSETS,        /* int32 [E_l + 1]   exclusive prefix of counts */
  MOE_WS_SORTED_TOK,     /* int32 [Npmax]     token of each pair, ascending within an expert */
  MOE_WS_SORTED_W,       /* fp32  [Npmax]     routing weight of each pair */
  MOE_WS_C,              /* bf16  [Npmax, I]  SwiGLU activations */
  MOE_WS_PARTIAL,        /* bf16  [T * (k - 1), H]  weighted GEMM2 rows of each token's 2nd..k-th
                            local pair (k = min(top_k, E_l)); the 1st goes straight into `out` */
  MOE_WS_CHUNK_COUNTS,   /* int32 [ceil(T/c), E_l] pairs per local expert per c-token group,
                            c = 4 for T <= 2048, else 16 (one row per routing workgroup) */
  MOE_WS_PAIR_DST,       /* int32 [Npmax]     GEMM2 destination of each pair: t (row of out) for
                            a token's first local pair, else -1 - (t * (k - 1) + j - 1) for its
                            (j+1)-th (row of partial) */
  MOE_WS_NUM_REGIONS     /* total size is written at this index */
};

/* Byte offsets of the regions above (offsets[MOE_WS_NUM_REGIONS] = total bytes). */
int moe_workspace_layout(const moe_geometry* geom, int T, int64_t* offsets);

/*
 * Stage timing hook. No counterpart in the reference's ABI; it plays the role of the reference's
 * compile-time MOE_TIMING phase counters (kda05_reproduction_single_shape/fable-5.1/moe_fp8_fwd/
 * t14107/moe_kernel.cu:39-52). With n == MOE_NUM_STAGES + 1, every later moe_run / moe_run_ex
 * records events[0] (hipEvent_t) before its first kernel and events[i] after stage i
 * (1 route, 2 permute, 3 GEMM1+SwiGLU, 4 GEMM2, 5 combine) on the call's stream; n == 0 turns
 * it off. Process-wide and not thread-safe: meant for benchmarks.
 */
#define MOE_NUM_STAGES 5
int moe_set_stage_events(void* const* events, int n);

/*
 * Activation quantisation, the step that produces `hs` / `hs_scale` for moe_run:
 * x bf16 [T, H] -> q e4m3fn [T, H], scale fp32 [H/128, T]. Per 1x128 block of a row,
 * scale = amax / 448 (0 for an all-zero block) and q = e4m3(clamp(x / s, -448, 448)) with
 * s = scale (1 when scale is 0), round to nearest even. H must be a multiple of 128.
 * Replaces: the per-row block quantisation the reference applies before its fp8 GEMM2
 *   (goal_full_shape/opus-4.8/moe_fp8_fwd/MOEDIR/main.py:151-156, same rule and constants)
 * and the hidden-state quantisation its harness performs to build `hidden_states_scale`.
 */
int moe_quantize_activations(const void* x, int T, int H, void* q, void* scale, void* stream);

/* Static description of a return code. */
const char* moe_error_string(int rc);

#ifdef __cplusplus
}
#endif
#endif /* JUSTGOAL_MOE_H */
