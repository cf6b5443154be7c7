// C ABI of the MoE operator (include/justgoal_moe.h): argument and geometry validation,
// workspace carving and the launch sequence route -> permute -> GEMM1+SwiGLU -> GEMM2 -> combine,
// all on the caller's stream. No host synchronisation, no allocation.
#include <hip/hip_runtime.h>

#include <mutex>
#include <string>

#include "justgoal_moe.h"
#include "moe_kernels.h"

namespace {

constexpr int64_t kAlign = 256;

const moe_geometry kDsV3 = {7168, 2048, 256, 32, 8, 8, 4, MOE_ROUTING_DS};

int64_t align_up(int64_t x) { return (x + kAlign - 1) / kAlign * kAlign; }

bool is_pow2(int x) { return x > 0 && (x & (x - 1)) == 0; }

// Geometry constraints of the kernels: 128-multiples for the scale blocks and the 128-column
// GEMM tiles, E a multiple of the wave width with at most 8 experts per lane, groups aligned to
// whole lanes in power-of-two lane counts, at most 8 selections.
int check_geometry(const moe_geometry* g) {
  if (!g) return MOE_ERR_INVALID_ARG;
  if (g->hidden <= 0 || g->hidden % 128 || g->hidden > 16384 || g->intermediate <= 0 ||
      g->intermediate % 128 || g->intermediate > 16384)
    return MOE_ERR_GEOMETRY;
  const int E = g->num_experts;
  if (E <= 0 || E % 64 || E > 512 || !is_pow2(E / 64)) return MOE_ERR_GEOMETRY;
  if (g->local_experts <= 0 || g->local_experts > E || g->local_experts > 256)
    return MOE_ERR_GEOMETRY;
  if (g->top_k <= 0 || g->top_k > 8 || g->top_k > E) return MOE_ERR_GEOMETRY;
  if (g->routing_method == MOE_ROUTING_DS) {
    if (g->n_group <= 0 || E % g->n_group) return MOE_ERR_GEOMETRY;
    const int gs = E / g->n_group, vpl = E / 64;
    if (gs < vpl || gs % vpl || !is_pow2(gs / vpl)) return MOE_ERR_GEOMETRY;
    if (g->topk_group <= 0 || g->topk_group > g->n_group) return MOE_ERR_GEOMETRY;
    if (g->top_k > g->topk_group * gs) return MOE_ERR_GEOMETRY;
  } else if (g->routing_method != MOE_ROUTING_SOFTMAX) {
    return MOE_ERR_GEOMETRY;
  }
  return MOE_OK;
}

// Local pairs a token can have: min(top_k, E_l).
int k_local(const moe_geometry* g) {
  return g->top_k < g->local_experts ? g->top_k : g->local_experts;
}

int64_t max_pairs(const moe_geometry* g, int T) { return (int64_t)T * k_local(g); }

// Most tokens one moe_run call takes. The kernels address activations, C rows and their scales
// with 32-bit buffer offsets: T*H must stay below the large-tile kernels' out-of-range marker
// (2^31 - 16) and max_pairs*I*2 (bytes of C) below 2^31. DS-V3: 65535 tokens.
int64_t token_limit(const moe_geometry* g) {
  const int64_t k = g->top_k < g->local_experts ? g->top_k : g->local_experts;
  const int64_t by_a = (int64_t)(0x7ffffff0 - 1) / g->hidden;
  const int64_t by_c = (int64_t)0x7fffffff / (k * g->intermediate * 2);
  return by_a < by_c ? by_a : by_c;
}

void layout(const moe_geometry* g, int T, int64_t* off) {
  const int64_t K = g->top_k, El = g->local_experts, Np = max_pairs(g, T);
  const int64_t sizes[MOE_WS_NUM_REGIONS] = {
      4 * T * K,                         // topk_idx
      4 * T * K,                         // topk_w
      4 * T * K,                         // pair_of
      4 * El,                            // counts
      4 * (El + 1),                      // offsets
      4 * Np,                            // sorted_tok
      4 * Np,                            // sorted_w
      2 * Np * g->intermediate,          // C (bf16)
      2 * (int64_t)T * (k_local(g) - 1) * g->hidden,  // partial (bf16, pairs 2.. of a token)
      4 * (int64_t)jgmoe::route_chunks(T) * El,  // chunk count rows
      4 * Np,                            // pair_dst
  };
  int64_t cur = 0;
  for (int i = 0; i < MOE_WS_NUM_REGIONS; ++i) {
    off[i] = cur;
    cur = align_up(cur + sizes[i]);
  }
  off[MOE_WS_NUM_REGIONS] = cur;
}

// The kernels use gfx950 instructions (f8f6f4 MFMA, scaled fp8 conversions); refuse other
// devices instead of faulting. Checked once per device.
int check_device() {
  static std::once_flag flags[64];
  static int status[64];
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return MOE_ERR_NO_DEVICE;
  std::call_once(flags[dev], [dev] {
    hipDeviceProp_t prop;
    if (hipGetDeviceProperties(&prop, dev) != hipSuccess) {
      status[dev] = MOE_ERR_NO_DEVICE;
      return;
    }
    status[dev] = (std::string(prop.gcnArchName).rfind("gfx950", 0) == 0) ? MOE_OK
                                                                          : MOE_ERR_NO_DEVICE;
  });
  return status[dev];
}

struct Regions {
  int32_t* topk_idx;
  float* topk_w;
  int32_t* pair_of;
  int32_t* counts;
  int32_t* offsets;
  int32_t* sorted_tok;
  float* sorted_w;
  uint16_t* C;
  uint16_t* partial;
  int32_t* hist;
  int32_t* pair_dst;
};

Regions carve(const moe_geometry* g, int T, void* ws) {
  int64_t off[MOE_WS_NUM_REGIONS + 1];
  layout(g, T, off);
  char* b = (char*)ws;
  return Regions{(int32_t*)(b + off[MOE_WS_TOPK_IDX]), (float*)(b + off[MOE_WS_TOPK_W]),
                 (int32_t*)(b + off[MOE_WS_PAIR_OF]),  (int32_t*)(b + off[MOE_WS_COUNTS]),
                 (int32_t*)(b + off[MOE_WS_OFFSETS]),  (int32_t*)(b + off[MOE_WS_SORTED_TOK]),
                 (float*)(b + off[MOE_WS_SORTED_W]),   (uint16_t*)(b + off[MOE_WS_C]),
                 (uint16_t*)(b + off[MOE_WS_PARTIAL]), (int32_t*)(b + off[MOE_WS_CHUNK_COUNTS]),
                 (int32_t*)(b + off[MOE_WS_PAIR_DST])};
}

#define JG_TRY(expr)                              \
  do {                                            \
    hipError_t e_ = (expr);                       \
    if (e_ != hipSuccess) return (int)e_;         \
  } while (0)

hipError_t mark_stage(int i, hipStream_t stream);

int route_and_permute(const moe_geometry* g, const void* logits, const void* bias,
                      int local_offset, float scaling, const Regions& r, int T,
                      hipStream_t stream) {
  JG_TRY(mark_stage(0, stream));
  JG_TRY(jgmoe::launch_route((const float*)logits, (const uint16_t*)bias, T, g->num_experts,
                             g->n_group, g->topk_group, g->top_k, g->routing_method, scaling,
                             local_offset, g->local_experts, r.topk_idx, r.topk_w, r.hist,
                             stream));
  JG_TRY(mark_stage(1, stream));
  JG_TRY(jgmoe::launch_permute(r.topk_idx, r.topk_w, r.hist, T, g->top_k, local_offset,
                               g->local_experts, r.counts, r.offsets, r.sorted_tok, r.sorted_w,
                               r.pair_dst, r.pair_of, stream));
  JG_TRY(mark_stage(2, stream));
  return MOE_OK;
}

// Scratch of moe_run_noalloc: one copy of this array per device, allocated by the runtime when
// the code object is loaded and held until the process ends. In host code `scratch` is only a
// host-side handle; the device address comes from hipGetSymbolAddress (scratch_ptr below).
static __device__ __align__(256) uint8_t scratch[MOE_NOALLOC_SCRATCH_BYTES];

constexpr int kMaxDevices = 64;
std::once_flag g_scratch_once[kMaxDevices];
void* g_scratch_ptr[kMaxDevices];
hipError_t g_scratch_status[kMaxDevices];

// Device address of this device's scratch array, looked up once per device with that device
// current. Returns the lookup's error code (and no pointer) if it failed.
hipError_t scratch_ptr(void** p) {
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return e;
  if (dev < 0 || dev >= kMaxDevices) return hipErrorInvalidDevice;
  std::call_once(g_scratch_once[dev], [dev] {
    void* q = nullptr;
    g_scratch_status[dev] = hipGetSymbolAddress(&q, HIP_SYMBOL(scratch));
    g_scratch_ptr[dev] = q;
  });
  if (g_scratch_status[dev] != hipSuccess) return g_scratch_status[dev];
  *p = g_scratch_ptr[dev];
  return hipSuccess;
}

hipEvent_t g_stage_events[MOE_NUM_STAGES + 1];
int g_stage_events_on = 0;

hipError_t mark_stage(int i, hipStream_t stream) {
  return g_stage_events_on ? hipEventRecord(g_stage_events[i], stream) : hipSuccess;
}

}  // namespace

extern "C" {

int moe_set_stage_events(void* const* events, int n) {
  if (n == 0) {
    g_stage_events_on = 0;
    return MOE_OK;
  }
  if (n != MOE_NUM_STAGES + 1 || !events) return MOE_ERR_INVALID_ARG;
  for (int i = 0; i < n; ++i) {
    if (!events[i]) return MOE_ERR_INVALID_ARG;
    g_stage_events[i] = (hipEvent_t)events[i];
  }
  g_stage_events_on = 1;
  return MOE_OK;
}

int64_t moe_workspace_bytes_ex(const moe_geometry* geom, int T) {
  const int rc = check_geometry(geom);
  if (rc != MOE_OK) return rc;
  if (T < 0) return MOE_ERR_INVALID_ARG;
  int64_t off[MOE_WS_NUM_REGIONS + 1];
  layout(geom, T, off);
  return off[MOE_WS_NUM_REGIONS];
}

int moe_workspace_bytes(int T) {
  const int64_t n = moe_workspace_bytes_ex(&kDsV3, T);
  return n > INT32_MAX ? MOE_ERR_INVALID_ARG : (int)n;
}

int moe_workspace_layout(const moe_geometry* geom, int T, int64_t* offsets) {
  const int rc = check_geometry(geom);
  if (rc != MOE_OK) return rc;
  if (T < 0 || !offsets) return MOE_ERR_INVALID_ARG;
  layout(geom, T, offsets);
  return MOE_OK;
}

int moe_route_ex(const moe_geometry* geom, const void* logits, const void* bias, int local_offset,
                 float scaling, void* workspace, int T, void* stream) {
  int rc = check_geometry(geom);
  if (rc != MOE_OK) return rc;
  if (T < 0) return MOE_ERR_INVALID_ARG;
  if (T == 0) return MOE_OK;
  if (!logits || !workspace) return MOE_ERR_INVALID_ARG;
  if ((rc = check_device()) != MOE_OK) return rc;
  return route_and_permute(geom, logits, bias, local_offset, scaling, carve(geom, T, workspace), T,
                           (hipStream_t)stream);
}

int moe_run_ex(const moe_geometry* geom, const void* logits, const void* bias, const void* hs,
               const void* hs_scale, const void* w13, const void* s13, const void* w2,
               const void* s2, int local_offset, float scaling, void* out, void* workspace, int T,
               void* stream_) {
  int rc = check_geometry(geom);
  if (rc != MOE_OK) return rc;
  if (T < 0 || T > token_limit(geom)) return MOE_ERR_INVALID_ARG;
  if (T == 0) return MOE_OK;
  if (!logits || !hs || !hs_scale || !w13 || !s13 || !w2 || !s2 || !out || !workspace)
    return MOE_ERR_INVALID_ARG;
  if ((rc = check_device()) != MOE_OK) return rc;
  hipStream_t stream = (hipStream_t)stream_;
  const Regions r = carve(geom, T, workspace);
  if ((rc = route_and_permute(geom, logits, bias, local_offset, scaling, r, T, stream)) != MOE_OK)
    return rc;
  const int H = geom->hidden, I = geom->intermediate, El = geom->local_experts;
  const int Np = (int)max_pairs(geom, T);
  const int rows_hint = (int)((int64_t)T * geom->top_k / geom->num_experts);
  JG_TRY(jgmoe::launch_gemm1((const uint8_t*)hs, (const float*)hs_scale, (const uint8_t*)w13,
                             (const float*)s13, r.counts, r.offsets, r.sorted_tok, r.C, T, H, I,
                             El, Np, rows_hint, stream));
  JG_TRY(mark_stage(3, stream));
  JG_TRY(jgmoe::launch_gemm2(r.C, (const uint8_t*)w2, (const float*)s2, r.counts, r.offsets,
                             r.sorted_w, jgmoe::Gemm2Out{r.pair_dst, (uint16_t*)out, r.partial},
                             H, I, El, Np, rows_hint, stream));
  JG_TRY(mark_stage(4, stream));
  JG_TRY(jgmoe::launch_combine(r.partial, r.pair_of, T, geom->top_k, k_local(geom), H,
                               (uint16_t*)out, stream));
  JG_TRY(mark_stage(5, stream));
  return MOE_OK;
}

int moe_run(const void* logits, const void* bias, const void* hs, const void* hs_scale,
            const void* w13, const void* s13, const void* w2, const void* s2, int local_offset,
            float scaling, void* out, void* workspace, int T, void* stream) {
  return moe_run_ex(&kDsV3, logits, bias, hs, hs_scale, w13, s13, w2, s2, local_offset, scaling,
                    out, workspace, T, stream);
}

int moe_run_noalloc(const moe_geometry* geom, const void* logits, const void* bias,
                    const void* hs, const void* hs_scale, const void* w13, const void* s13,
                    const void* w2, const void* s2, int local_offset, float scaling, void* out,
                    int T, void* stream) {
  int rc = check_geometry(geom);
  if (rc != MOE_OK) return rc;
  if (T < 0) return MOE_ERR_INVALID_ARG;
  if (T == 0) return MOE_OK;
  int64_t off[MOE_WS_NUM_REGIONS + 1];
  layout(geom, T, off);
  if (off[MOE_WS_NUM_REGIONS] > (int64_t)MOE_NOALLOC_SCRATCH_BYTES) return MOE_ERR_SCRATCH_SIZE;
  if ((rc = check_device()) != MOE_OK) return rc;
  void* ws = nullptr;
  JG_TRY(scratch_ptr(&ws));
  // No region of the workspace has to start at any value (every kernel writes before it reads),
  // so the scratch array is used as it is, left over from the previous call.
  return moe_run_ex(geom, logits, bias, hs, hs_scale, w13, s13, w2, s2, local_offset, scaling,
                    out, ws, T, stream);
}

int moe_quantize_activations(const void* x, int T, int H, void* q, void* scale, void* stream) {
  if (T < 0 || H <= 0 || H % 128 != 0) return MOE_ERR_INVALID_ARG;
  if (T == 0) return MOE_OK;
  if (!x || !q || !scale) return MOE_ERR_INVALID_ARG;
  const int rc = check_device();
  if (rc != MOE_OK) return rc;
  JG_TRY(jgmoe::launch_quantize_activations((const uint16_t*)x, T, H, (uint8_t*)q, (float*)scale,
                                            (hipStream_t)stream));
  return MOE_OK;
}

const char* moe_error_string(int rc) {
  switch (rc) {
    case MOE_OK: return "success";
    case MOE_ERR_INVALID_ARG:
      return "invalid argument (null pointer, negative token count, or more tokens than one call "
             "takes)";
    case MOE_ERR_GEOMETRY: return "unsupported MoE geometry";
    case MOE_ERR_NO_DEVICE: return "no gfx950 (MI355X) device is current";
    case MOE_ERR_SCRATCH_SIZE:
      return "the call needs more workspace than moe_run_noalloc's fixed scratch array holds "
             "(use moe_run_ex with a caller workspace)";
    default: return rc > 0 ? hipGetErrorString((hipError_t)rc) : "unknown error";
  }
}

}  // extern "C"
