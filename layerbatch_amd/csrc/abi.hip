// C ABI of liblbmoe (include/lbmoe.h): argument validation, workspace layout and the stage
// order of the MoE block. The Python module layerbatch_amd.moe binds these entry points; the
// reference module they replace is Qwen3_5SparseMoeBlock (nanovllm/models/qwen3_5.py:881-917).
#include <hip/hip_runtime.h>

#include <algorithm>
#include <atomic>
#include <cstring>

#include "internal.hpp"

namespace lbmoe {

static size_t align256(size_t v) { return (v + 255) & ~static_cast<size_t>(255); }

static bool is_fp8(const lbmoe_layer& L) { return L.weight_dtype == LBMOE_W_FP8_E4M3; }

WsLayout ws_layout(const lbmoe_layer& L, int64_t T) {
  const int64_t E = L.num_experts, k = L.top_k, H = L.hidden_size;
  const int64_t I = L.moe_intermediate_size, Is = L.shared_intermediate_size;
  const int64_t V = T * k, Vs = V + (Is > 0 ? T : 0), Imax = std::max(I, Is);
  // count chunks: kPermChunk entries (launch_permute) or slot x 64-token block (router_route)
  const int64_t nblk = std::max(perm_blocks(V), router_route_chunks(T, static_cast<int>(k)));
  WsLayout w{};
  w.bytes[R_LOGITS] = T * E * 2;
  w.bytes[R_IDX] = V * 4;
  w.bytes[R_TOPW] = V * 2;
  w.bytes[R_SGATE] = T * 4;
  w.bytes[R_COUNTS] = (E + 1) * 4;
  w.bytes[R_OFFSETS] = (E + 2) * 4;
  w.bytes[R_PERM_TOK] = Vs * 4;
  w.bytes[R_PERM_SLOT] = V * 4;
  w.bytes[R_INV] = V * 4;
  w.bytes[R_ACT] = Vs * Imax * 2;
  w.bytes[R_OUT] = Vs * H * 2;
  w.bytes[R_XN] = T * H * 2;
  w.bytes[R_HIST] = E * nblk * 4;
  w.bytes[R_BASE] = E * nblk * 4;
  w.bytes[R_LRANK] = V * 4;
  w.bytes[R_TILES] = tiled_list_bytes(tiled_max_tiles(Vs, E + 1), L.moe_intermediate_size,
                                      L.shared_intermediate_size, H);
  if (is_fp8(L)) {
    w.bytes[R_XQ] = T * H;
    // the scale regions end in 16 spare bytes: the tiled fp8 GEMMs copy a row's scales in
    // 16-byte pieces, whose last may reach 12 bytes past the final row
    w.bytes[R_XS] = T * (H / 128) * 4 + 16;
    w.bytes[R_ACTQ] = Vs * Imax;
    w.bytes[R_ACTS] = Vs * (Imax / 128) * 4 + 16;
  }
  size_t off = 0;
  for (int r = 0; r < R_COUNT_; ++r) {
    w.off[r] = off;
    off += align256(w.bytes[r]);
  }
  w.total = off;
  return w;
}

void perm_scratch_layout(int64_t T, int k, int E, size_t* hist_off, size_t* base_off,
                         size_t* lrank_off, size_t* total) {
  const int64_t V = T * k, nblk = perm_blocks(V);
  *hist_off = 0;
  *base_off = align256(E * nblk * 4);
  *lrank_off = *base_off + align256(E * nblk * 4);
  *total = *lrank_off + align256(V * 4);
}

static int32_t check_device() {
  static std::atomic<int> cache[64];   // per device: 0 unknown, 1 gfx950, 2 other
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return LBMOE_ERR_DEVICE;
  int c = cache[dev].load(std::memory_order_relaxed);
  if (c == 0) {
    hipDeviceProp_t prop;
    if (hipGetDeviceProperties(&prop, dev) != hipSuccess) return LBMOE_ERR_DEVICE;
    c = std::strncmp(prop.gcnArchName, "gfx950", 6) == 0 ? 1 : 2;
    cache[dev].store(c, std::memory_order_relaxed);
  }
  return c == 1 ? LBMOE_OK : LBMOE_ERR_DEVICE;
}

static int32_t check_shape(const lbmoe_layer* layer) {
  if (layer == nullptr) return LBMOE_ERR_NULL;
  const lbmoe_layer& L = *layer;
  if (L.hidden_size <= 0 || L.hidden_size % 128 != 0 || L.hidden_size > 65536)
    return LBMOE_ERR_SHAPE;
  if (L.num_experts < 1 || L.num_experts > 1024) return LBMOE_ERR_SHAPE;
  if (L.top_k < 1 || L.top_k > 32 || L.top_k > L.num_experts) return LBMOE_ERR_SHAPE;
  if (L.moe_intermediate_size <= 0 || L.moe_intermediate_size % 128 != 0 ||
      L.moe_intermediate_size > 65536)
    return LBMOE_ERR_SHAPE;
  if (L.shared_intermediate_size < 0 || L.shared_intermediate_size % 128 != 0 ||
      L.shared_intermediate_size > 65536)
    return LBMOE_ERR_SHAPE;
  if (L.weight_dtype != LBMOE_W_BF16 && L.weight_dtype != LBMOE_W_FP8_E4M3)
    return LBMOE_ERR_DTYPE;
  // fp8 kernels stream 256-byte (= 256 k) row segments holding two 128-k scale blocks
  if (L.weight_dtype == LBMOE_W_FP8_E4M3 &&
      (L.hidden_size % 256 != 0 || L.moe_intermediate_size % 256 != 0 ||
       L.shared_intermediate_size % 256 != 0))
    return LBMOE_ERR_SHAPE;
  return LBMOE_OK;
}

static int32_t check_expert_ptrs(const lbmoe_layer& L) {
  if (!L.gate_up_proj || !L.down_proj) return LBMOE_ERR_NULL;
  if (is_fp8(L) && (!L.gate_up_scale || !L.down_scale)) return LBMOE_ERR_NULL;
  return LBMOE_OK;
}

static int32_t check_shared_ptrs(const lbmoe_layer& L) {
  if (!L.shared_gate_proj || !L.shared_up_proj || !L.shared_down_proj || !L.shared_expert_gate)
    return LBMOE_ERR_NULL;
  if (is_fp8(L) && (!L.shared_gate_scale || !L.shared_up_scale || !L.shared_down_scale))
    return LBMOE_ERR_NULL;
  return LBMOE_OK;
}

static int32_t check_T(const lbmoe_layer& L, int64_t T) {
  if (T < 0 || T > (int64_t{1} << 21)) return LBMOE_ERR_SHAPE;
  if (T * (L.top_k + 1) > INT32_MAX) return LBMOE_ERR_SHAPE;
  return LBMOE_OK;
}

static GroupWeights group_weights(const lbmoe_layer& L, bool with_shared, int64_t T) {
  GroupWeights g{};
  g.gate_up = L.gate_up_proj;
  g.down = L.down_proj;
  g.gate_up_scale = L.gate_up_scale;
  g.down_scale = L.down_scale;
  g.sh_gate = L.shared_gate_proj;
  g.sh_up = L.shared_up_proj;
  g.sh_down = L.shared_down_proj;
  g.sh_gate_scale = L.shared_gate_scale;
  g.sh_up_scale = L.shared_up_scale;
  g.sh_down_scale = L.shared_down_scale;
  g.gate_up_tiled = L.gate_up_tiled;
  g.down_tiled = L.down_tiled;
  g.sh_gate_up_tiled = L.shared_gate_up_tiled;
  g.sh_down_tiled = L.shared_down_tiled;
  g.E = L.num_experts;
  g.H = L.hidden_size;
  g.I = L.moe_intermediate_size;
  g.Is = L.shared_intermediate_size;
  g.g0 = 0;
  g.groups = L.num_experts + (with_shared ? 1 : 0);
  g.sh_row0 = static_cast<int>(T * L.top_k);
  return g;
}

template <typename P>
static P* at(void* ws, const WsLayout& w, int r) {
  return reinterpret_cast<P*>(static_cast<char*>(ws) + w.off[r]);
}

#define LBMOE_TRY(expr)                                       \
  do {                                                        \
    if ((expr) != hipSuccess) return LBMOE_ERR_LAUNCH;        \
  } while (0)

// Expected tokens per routed expert at which the LDS-tiled GEMMs replace weight streaming.
// Measured (back-to-back µs per layer call): at 24 tokens per expert both are even
// (Qwen3-30B-A3B T=384: 286-291); from 30 on the tiled GEMMs win clearly (T=512: 293 vs 431,
// E=512 T=1536: 731 vs 998), the streaming kernels then needing four token tiles per pass;
// at 20 streaming wins (E=512 T=1024: 672 vs 714, fp8 427 vs 484).
constexpr double kTiledMinTokensPerExpert = 28.0;

static bool use_tiled(const GroupWeights& gw, int64_t T, int k) {
  return tiled_supported(gw) && tiled_offsets_fit(gw, T, k) &&
         static_cast<double>(T) * k / gw.E >= kTiledMinTokensPerExpert;
}

// Routed experts of one call: permute, gate_up, down, combine.
// Optional instrumentation: when ev is non-null, ev->mark(s) records the next event after
// each stage.
struct StageEvents {
  void* const* events;
  int n;
  int next;
  hipError_t mark(hipStream_t s) {
    if (!events || next >= n) return hipSuccess;
    return hipEventRecord(static_cast<hipEvent_t>(events[next++]), s);
  }
};

// rt: the batch's routing runs inside the gate_up kernel (launch_gate_up_bf16_routed), which
// also writes the permutation; only for bf16 weights and the weight-streaming GEMMs.
// chunked: the route came from launch_router_route, whose per-chunk counts (R_HIST, R_LRANK)
// the permutation finishes (scan, then scatter with the tile list).
static int32_t run_experts(const lbmoe_layer& L, const void* x, const void* idx, int idx_bytes,
                           const void* topw, const float* sgate, int64_t T, void* y, void* ws,
                           const WsLayout& w, bool with_shared, hipStream_t s,
                           StageEvents* ev = nullptr, bool permuted = false,
                           const SmallRoute* rt = nullptr, bool own_ids = false,
                           bool chunked = false, bool x_quantised = false) {
  StageEvents none{nullptr, 0, 0};
  if (!ev) ev = &none;
  const int k = L.top_k, E = L.num_experts, H = L.hidden_size;
  const int Imax = std::max(L.moe_intermediate_size, L.shared_intermediate_size);
  int32_t* counts = at<int32_t>(ws, w, R_COUNTS);
  int32_t* offsets = at<int32_t>(ws, w, R_OFFSETS);
  int32_t* perm_tok = at<int32_t>(ws, w, R_PERM_TOK);
  int32_t* inv = at<int32_t>(ws, w, R_INV);
  GroupWeights gw = group_weights(L, with_shared, T);
  // the weight-streaming GEMMs give workgroups only to the at most T*k experts with tokens
  if (T * k < E) gw.hit_rows = static_cast<int>(T * k);
  // the route's own ids (all in [0, E)) can be permuted inside the bf16 decode gate_up kernel
  const bool perm_in_gate_up = own_ids && !permuted && idx_bytes == 4 && !is_fp8(L) &&
                               !use_tiled(gw, T, k) && gate_up_perm_supported(gw, T, k);
  int32_t* tiles = at<int32_t>(ws, w, R_TILES);
  const int max_tiles = tiled_max_tiles(T * k + (with_shared ? T : 0), gw.groups);
  bool tiles_built = false;
  if (chunked) {
    int32_t* base = at<int32_t>(ws, w, R_BASE);
    LBMOE_TRY(launch_perm_scan(at<int32_t>(ws, w, R_HIST),
                               static_cast<int>(router_route_chunks(T, k)), E, base, counts, s));
    LBMOE_TRY(launch_scatter_build(static_cast<const int32_t*>(idx), T, k, base, counts,
                                   at<int32_t>(ws, w, R_LRANK), offsets, perm_tok,
                                   at<int32_t>(ws, w, R_PERM_SLOT), inv, gw, with_shared,
                                   max_tiles, tiles, s));
    tiles_built = true;
  } else if (!permuted && !perm_in_gate_up) {
    const bool tiled = use_tiled(gw, T, k) &&
                       (!is_fp8(L) || tiled_fp8_supported(gw, T, T * k + (with_shared ? T : 0)));
    if (tiled && perm_chunked(T * k, E)) {
      // prefill GEMMs: the permutation's scatter and the tile list in one launch
      int32_t* base = at<int32_t>(ws, w, R_BASE);
      int32_t* lrank = at<int32_t>(ws, w, R_LRANK);
      LBMOE_TRY(launch_perm_count_scan(idx, idx_bytes, T, k, E, at<int32_t>(ws, w, R_HIST), base,
                                       lrank, counts, s));
      LBMOE_TRY(launch_perm_scatter_build(idx, idx_bytes, T, k, base, counts, lrank, offsets,
                                          perm_tok, at<int32_t>(ws, w, R_PERM_SLOT), inv, gw,
                                          with_shared, max_tiles, tiles, s));
      tiles_built = true;
    } else {
      LBMOE_TRY(launch_permute(idx, idx_bytes, T, k, E, with_shared, counts, offsets, perm_tok,
                               at<int32_t>(ws, w, R_PERM_SLOT), inv, at<int32_t>(ws, w, R_HIST),
                               at<int32_t>(ws, w, R_BASE), at<int32_t>(ws, w, R_LRANK), s));
    }
  }
  LBMOE_TRY(ev->mark(s));
  void* act = at<void>(ws, w, R_ACT);
  void* out = at<void>(ws, w, R_OUT);
  if (is_fp8(L)) {
    // fp8: activations quantised per (row, 128 channels) before each GEMM
    void* xq = at<void>(ws, w, R_XQ);
    float* xs = at<float>(ws, w, R_XS);
    void* actq = at<void>(ws, w, R_ACTQ);
    float* acts = at<float>(ws, w, R_ACTS);
    const int64_t rows = T * k + (with_shared ? T : 0);
    if (!x_quantised) LBMOE_TRY(launch_quant_groups_fp8(x, T, H, H, xq, xs, s));
    if (use_tiled(gw, T, k) && tiled_fp8_supported(gw, T, rows)) {
      if (!tiles_built)
        LBMOE_TRY(launch_build_tiles(counts, offsets, gw, with_shared, T, max_tiles, tiles, s));
      LBMOE_TRY(launch_gate_up_tiled_fp8(gw, xq, xs, perm_tok, tiles, max_tiles, Imax, actq, acts,
                                         s));
      LBMOE_TRY(ev->mark(s));
      LBMOE_TRY(launch_down_tiled_fp8(gw, actq, acts, Imax, tiles, max_tiles, out, s));
    } else {
      LBMOE_TRY(launch_gate_up_fp8(gw, xq, xs, counts, offsets, perm_tok, T, k, Imax, act, s));
      LBMOE_TRY(ev->mark(s));
      LBMOE_TRY(launch_quant_groups_fp8(act, rows, Imax, Imax, actq, acts, s));
      LBMOE_TRY(launch_down_fp8(gw, actq, acts, Imax, counts, offsets, T, k, out, s));
    }
    LBMOE_TRY(ev->mark(s));
    LBMOE_TRY(launch_combine(out, inv, topw, sgate, T, k, H, with_shared, y, s));
    LBMOE_TRY(ev->mark(s));
    return LBMOE_OK;
  }
  if (rt && use_tiled(gw, T, k)) return LBMOE_ERR_SHAPE;   // not reached (see forward_impl)
  if (use_tiled(gw, T, k)) {
    // prefill-sized batch: LDS-tiled MFMA GEMMs over a device-built token-tile list
    if (!tiles_built)
      LBMOE_TRY(launch_build_tiles(counts, offsets, gw, with_shared, T, max_tiles, tiles, s));
    LBMOE_TRY(launch_gate_up_tiled(gw, x, perm_tok, tiles, max_tiles, T, Imax, act, s));
    LBMOE_TRY(ev->mark(s));
    LBMOE_TRY(launch_down_tiled(gw, act, Imax, tiles, max_tiles, T, out, s));
  } else {
    if (rt) {
      LBMOE_TRY(launch_gate_up_bf16_routed(gw, x, *rt, T, Imax, act, s));
    } else if (perm_in_gate_up) {
      const PermOut po{counts, offsets, perm_tok, at<int32_t>(ws, w, R_PERM_SLOT), inv};
      LBMOE_TRY(launch_gate_up_bf16_perm(gw, x, static_cast<const int32_t*>(idx), po, T, k,
                                         Imax, act, s));
    } else {
      LBMOE_TRY(launch_gate_up_bf16(gw, x, counts, offsets, perm_tok, T, k, Imax, act, s));
    }
    LBMOE_TRY(ev->mark(s));
    if (idx_bytes == 4 && down_combine_small_supported(gw, T, k)) {
      // one launch for the down GEMM and the combine (profiled: the combine stage is empty)
      LBMOE_TRY(launch_down_combine_small(gw, act, Imax, static_cast<const int32_t*>(idx), inv,
                                          topw, sgate, T, k, with_shared, y, s));
      LBMOE_TRY(ev->mark(s));
      LBMOE_TRY(ev->mark(s));
      return LBMOE_OK;
    }
    LBMOE_TRY(launch_down_bf16(gw, act, Imax, counts, offsets, T, k, out, s));
  }
  LBMOE_TRY(ev->mark(s));
  LBMOE_TRY(launch_combine(out, inv, topw, sgate, T, k, H, with_shared, y, s));
  LBMOE_TRY(ev->mark(s));
  return LBMOE_OK;
}

}  // namespace lbmoe

using namespace lbmoe;

extern "C" {

const char* lbmoe_status_string(int32_t status) {
  switch (status) {
    case LBMOE_OK: return "ok";
    case LBMOE_ERR_NULL: return "required pointer is NULL";
    case LBMOE_ERR_SHAPE: return "unsupported or inconsistent shape";
    case LBMOE_ERR_DTYPE: return "unsupported dtype or index width";
    case LBMOE_ERR_WORKSPACE: return "workspace too small";
    case LBMOE_ERR_DEVICE: return "current device is not gfx950";
    case LBMOE_ERR_LAUNCH: return "kernel launch failed";
    case LBMOE_ERR_STATIC_LIMIT:
      return "call needs more workspace than the static workspace holds "
             "(LBMOE_STATIC_WORKSPACE_BYTES)";
    default: return "unknown status";
  }
}

int32_t lbmoe_abi_version(void) { return LBMOE_ABI_VERSION; }

int32_t lbmoe_check_layer(const lbmoe_layer* layer) {
  int32_t st = check_shape(layer);
  if (st != LBMOE_OK) return st;
  const lbmoe_layer& L = *layer;
  if (!L.gate_weight) return LBMOE_ERR_NULL;
  if ((st = check_expert_ptrs(L)) != LBMOE_OK) return st;
  if (is_fp8(L) && (L.gate_up_tiled || L.down_tiled || L.shared_gate_up_tiled ||
                    L.shared_down_tiled))
    return LBMOE_ERR_DTYPE;             // the tiled copies are bf16 layouts
  if (L.shared_intermediate_size > 0) return check_shared_ptrs(L);
  return LBMOE_OK;
}

int32_t lbmoe_pack_weights(const lbmoe_layer* layer, void* gate_up_tiled, void* down_tiled,
                           void* shared_gate_up_tiled, void* shared_down_tiled, void* stream) {
  int32_t st = lbmoe_check_layer(layer);
  if (st != LBMOE_OK) return st;
  const lbmoe_layer& L = *layer;
  if (is_fp8(L)) return LBMOE_ERR_DTYPE;
  const bool sh = L.shared_intermediate_size > 0;
  if (!gate_up_tiled || !down_tiled || (sh && (!shared_gate_up_tiled || !shared_down_tiled)))
    return LBMOE_ERR_NULL;
  if (!tiled_supported(group_weights(L, sh, 0))) return LBMOE_ERR_SHAPE;
  if ((st = check_device()) != LBMOE_OK) return st;
  hipStream_t s = static_cast<hipStream_t>(stream);
  const int E = L.num_experts, H = L.hidden_size, I = L.moe_intermediate_size;
  const int Is = L.shared_intermediate_size;
  const auto* gu = static_cast<const uint16_t*>(L.gate_up_proj);
  LBMOE_TRY(launch_pack_tiled(gu, gu + static_cast<int64_t>(I) * H, int64_t{2} * I * H, E, I, H,
                              true, static_cast<uint16_t*>(gate_up_tiled), s));
  LBMOE_TRY(launch_pack_tiled(static_cast<const uint16_t*>(L.down_proj), nullptr,
                              static_cast<int64_t>(H) * I, E, H, I, false,
                              static_cast<uint16_t*>(down_tiled), s));
  if (sh) {
    LBMOE_TRY(launch_pack_tiled(static_cast<const uint16_t*>(L.shared_gate_proj),
                                static_cast<const uint16_t*>(L.shared_up_proj), 0, 1, Is, H, true,
                                static_cast<uint16_t*>(shared_gate_up_tiled), s));
    LBMOE_TRY(launch_pack_tiled(static_cast<const uint16_t*>(L.shared_down_proj), nullptr, 0, 1,
                                H, Is, false, static_cast<uint16_t*>(shared_down_tiled), s));
  }
  return LBMOE_OK;
}

int32_t lbmoe_workspace_size(const lbmoe_layer* layer, int64_t T, size_t* bytes) {
  if (!bytes) return LBMOE_ERR_NULL;
  int32_t st = check_shape(layer);
  if (st != LBMOE_OK) return st;
  if ((st = check_T(*layer, T)) != LBMOE_OK) return st;
  *bytes = ws_layout(*layer, T).total;
  return LBMOE_OK;
}

int32_t lbmoe_workspace_region(const lbmoe_layer* layer, int64_t T, int32_t region,
                               size_t* offset, size_t* bytes) {
  if (!offset || !bytes) return LBMOE_ERR_NULL;
  int32_t st = check_shape(layer);
  if (st != LBMOE_OK) return st;
  if ((st = check_T(*layer, T)) != LBMOE_OK) return st;
  if (region < 0 || region >= kPublicRegions) return LBMOE_ERR_SHAPE;
  const WsLayout w = ws_layout(*layer, T);
  *offset = w.off[region];
  *bytes = w.bytes[region];
  return LBMOE_OK;
}

}  // extern "C"

namespace lbmoe {

// The decoder layer's residual add + RMSNorm ahead of the block (lbmoe_forward_norm).
struct NormArgs {
  const void* residual;
  const void* weight;
  float eps;
  void* residual_out;
};

// Whether the block routes through launch_router_route: the tiled router over at most 128
// experts, with the tiled expert GEMMs after it (their tile list is built with the scatter).
static bool route_in_router(const lbmoe_layer& L, int64_t T, bool sh) {
  const int E = L.num_experts, H = L.hidden_size, k = L.top_k;
  if (!router_is_tiled(T, E, H) || !router_route_supported(E, H, k)) return false;
  const GroupWeights gw = group_weights(L, sh, T);
  if (!use_tiled(gw, T, k)) return false;
  return !is_fp8(L) || tiled_fp8_supported(gw, T, T * k + (sh ? T : 0));
}

static int32_t forward_impl(const lbmoe_layer* layer, const void* x, int64_t T, void* y,
                            void* workspace, size_t workspace_bytes, void* stream,
                            StageEvents* ev, const NormArgs* norm = nullptr) {
  int32_t st = lbmoe_check_layer(layer);
  if (st != LBMOE_OK) return st;
  const lbmoe_layer& L = *layer;
  if ((st = check_T(L, T)) != LBMOE_OK) return st;
  if (T == 0) return LBMOE_OK;
  if (!x || !y || !workspace) return LBMOE_ERR_NULL;
  const WsLayout w = ws_layout(L, T);
  if (workspace_bytes < w.total) return LBMOE_ERR_WORKSPACE;
  if ((st = check_device()) != LBMOE_OK) return st;
  hipStream_t s = static_cast<hipStream_t>(stream);
  void* ws = workspace;
  const bool sh = L.shared_intermediate_size > 0;
  void* logits = at<void>(ws, w, R_LOGITS);
  void* idx = at<void>(ws, w, R_IDX);
  void* topw = at<void>(ws, w, R_TOPW);
  float* sgate = sh ? at<float>(ws, w, R_SGATE) : nullptr;
  LBMOE_TRY(ev->mark(s));
  if (!norm && route_in_router(L, T, sh)) {
    // logits, selection and the permutation's count pass in one launch, or two with the k range
    // split (profiled calls time it as the router stage, the routing stage then being empty);
    // the split's partial sums go to the expert-output region, which only the down GEMM writes
    LBMOE_TRY(launch_router_route(x, L.gate_weight, L.logit_bias, L.shared_expert_gate, T,
                                  L.num_experts, L.hidden_size, L.top_k, logits,
                                  static_cast<int32_t*>(idx), topw, sgate,
                                  at<int32_t>(ws, w, R_HIST), at<int32_t>(ws, w, R_LRANK),
                                  at<void>(ws, w, R_OUT), w.bytes[R_OUT], s));
    LBMOE_TRY(ev->mark(s));
    LBMOE_TRY(ev->mark(s));
    return run_experts(L, x, idx, 4, topw, sgate, T, y, ws, w, sh, s, ev, false, nullptr, true,
                       true);
  }
  if (norm) {
    // x is the attention output: the block's input is the normalised residual sum
    void* xn = at<void>(ws, w, R_XN);
    LBMOE_TRY(launch_add_rmsnorm_router(x, norm->residual, norm->weight, norm->eps, L.gate_weight,
                                        T, L.num_experts, L.hidden_size, logits, xn,
                                        norm->residual_out, s));
    x = xn;
  } else {
    LBMOE_TRY(launch_router_logits(x, L.gate_weight, T, L.num_experts, L.hidden_size, logits, s));
  }
  LBMOE_TRY(ev->mark(s));
  // the smallest bf16 batches route inside the gate_up kernel (profiled calls then have
  // empty routing and permutation stages; T*k/E <= 4 tokens per expert never reaches the
  // tiled GEMMs)
  if (!is_fp8(L) && inline_route_supported(T, L.top_k, L.num_experts)) {
    const SmallRoute rt{static_cast<const uint16_t*>(logits), L.logit_bias,
                        static_cast<const uint16_t*>(L.shared_expert_gate), L.top_k,
                        static_cast<int32_t*>(idx), static_cast<uint16_t*>(topw), sgate,
                        at<int32_t>(ws, w, R_COUNTS), at<int32_t>(ws, w, R_OFFSETS),
                        at<int32_t>(ws, w, R_PERM_TOK), at<int32_t>(ws, w, R_PERM_SLOT),
                        at<int32_t>(ws, w, R_INV)};
    LBMOE_TRY(ev->mark(s));
    return run_experts(L, x, idx, 4, topw, sgate, T, y, ws, w, sh, s, ev, true, &rt);
  }
  // small batches route and permute in one kernel (profiled calls time it as the routing
  // stage, their permutation stage then being empty)
  if (route_perm_small_supported(T, L.top_k, L.num_experts)) {
    LBMOE_TRY(launch_route_perm_small(
        logits, L.logit_bias, x, L.shared_expert_gate, T, L.num_experts, L.hidden_size, L.top_k,
        static_cast<int32_t*>(idx), topw, sgate, at<int32_t>(ws, w, R_COUNTS),
        at<int32_t>(ws, w, R_OFFSETS), at<int32_t>(ws, w, R_PERM_TOK),
        at<int32_t>(ws, w, R_PERM_SLOT), at<int32_t>(ws, w, R_INV), s));
    LBMOE_TRY(ev->mark(s));
    return run_experts(L, x, idx, 4, topw, sgate, T, y, ws, w, sh, s, ev, true);
  }
  // fp8 layers with a shared expert: the selection kernel, which reads x for the shared gate,
  // also writes x's e4m3 codes and scales
  const bool fuse_q = is_fp8(L) && sh;
  LBMOE_TRY(launch_route_topk(logits, L.logit_bias, x, L.shared_expert_gate, T, L.num_experts,
                              L.hidden_size, L.top_k, idx, 4, topw, sgate, s,
                              fuse_q ? at<void>(ws, w, R_XQ) : nullptr,
                              fuse_q ? at<float>(ws, w, R_XS) : nullptr));
  LBMOE_TRY(ev->mark(s));
  return run_experts(L, x, idx, 4, topw, sgate, T, y, ws, w, sh, s, ev, false, nullptr, true,
                     false, fuse_q);
}

}  // namespace lbmoe

extern "C" {

int32_t lbmoe_forward(const lbmoe_layer* layer, const void* x, int64_t T, void* y,
                      void* workspace, size_t workspace_bytes, void* stream) {
  StageEvents none{nullptr, 0, 0};
  return forward_impl(layer, x, T, y, workspace, workspace_bytes, stream, &none);
}

int32_t lbmoe_forward_profiled(const lbmoe_layer* layer, const void* x, int64_t T, void* y,
                               void* workspace, size_t workspace_bytes, void* stream,
                               void* const* events, int32_t n_events) {
  if (!events || n_events < LBMOE_PROFILE_EVENTS) return LBMOE_ERR_NULL;
  StageEvents ev{events, n_events, 0};
  return forward_impl(layer, x, T, y, workspace, workspace_bytes, stream, &ev);
}

int32_t lbmoe_forward_norm(const lbmoe_layer* layer, const void* hidden, const void* residual,
                           const void* norm_weight, float eps, int64_t T, void* y,
                           void* residual_out, void* workspace, size_t workspace_bytes,
                           void* stream) {
  if (T > 0 && (!hidden || !residual || !norm_weight || !residual_out)) return LBMOE_ERR_NULL;
  // the fused router reads residual rows in several workgroups while others write residual_out
  if (T > 0 && residual_out == residual) return LBMOE_ERR_SHAPE;
  if (!(eps >= 0.f)) return LBMOE_ERR_SHAPE;
  StageEvents none{nullptr, 0, 0};
  const NormArgs norm{residual, norm_weight, eps, residual_out};
  return forward_impl(layer, hidden, T, y, workspace, workspace_bytes, stream, &none, &norm);
}

int32_t lbmoe_router_logits(const lbmoe_layer* layer, const void* x, int64_t T, void* logits,
                            void* stream) {
  int32_t st = check_shape(layer);
  if (st != LBMOE_OK) return st;
  if (!layer->gate_weight) return LBMOE_ERR_NULL;
  if ((st = check_T(*layer, T)) != LBMOE_OK) return st;
  if (T == 0) return LBMOE_OK;
  if (!x || !logits) return LBMOE_ERR_NULL;
  if ((st = check_device()) != LBMOE_OK) return st;
  LBMOE_TRY(launch_router_logits(x, layer->gate_weight, T, layer->num_experts,
                                 layer->hidden_size, logits, static_cast<hipStream_t>(stream)));
  return LBMOE_OK;
}

int32_t lbmoe_route(const lbmoe_layer* layer, const void* logits, const void* x, int64_t T,
                    void* topk_idx, int32_t idx_bytes, void* topk_w, float* shared_gate,
                    void* stream) {
  int32_t st = check_shape(layer);
  if (st != LBMOE_OK) return st;
  if ((st = check_T(*layer, T)) != LBMOE_OK) return st;
  if (idx_bytes != 4 && idx_bytes != 8) return LBMOE_ERR_DTYPE;
  if (T == 0) return LBMOE_OK;
  if (!logits || !topk_idx || !topk_w) return LBMOE_ERR_NULL;
  const bool gate = shared_gate != nullptr;
  if (gate && (!x || !layer->shared_expert_gate)) return LBMOE_ERR_NULL;
  if ((st = check_device()) != LBMOE_OK) return st;
  LBMOE_TRY(launch_route_topk(logits, layer->logit_bias, x, layer->shared_expert_gate, T,
                              layer->num_experts, layer->hidden_size, layer->top_k, topk_idx,
                              idx_bytes, topk_w, shared_gate, static_cast<hipStream_t>(stream)));
  return LBMOE_OK;
}

int32_t lbmoe_permute_workspace_size(int64_t T, int32_t k, int32_t E, size_t* bytes) {
  if (!bytes) return LBMOE_ERR_NULL;
  if (T < 0 || k < 1 || k > 32 || E < 1 || E > 1024 || k > E || T * k > INT32_MAX)
    return LBMOE_ERR_SHAPE;
  size_t h, b, l;
  perm_scratch_layout(T, k, E, &h, &b, &l, bytes);
  return LBMOE_OK;
}

int32_t lbmoe_permute(const void* topk_idx, int32_t idx_bytes, int64_t T, int32_t k,
                      int32_t E, int32_t* counts, int32_t* offsets, int32_t* perm_tok,
                      int32_t* perm_slot, int32_t* inv, void* workspace,
                      size_t workspace_bytes, void* stream) {
  if (idx_bytes != 4 && idx_bytes != 8) return LBMOE_ERR_DTYPE;
  if (T < 0 || k < 1 || k > 32 || E < 1 || E > 1024 || k > E || T * k > INT32_MAX)
    return LBMOE_ERR_SHAPE;
  if (!counts || !offsets) return LBMOE_ERR_NULL;
  size_t h, b, l, total;
  perm_scratch_layout(T, k, E, &h, &b, &l, &total);
  if (T > 0 && (!topk_idx || !perm_tok || !perm_slot || !inv)) return LBMOE_ERR_NULL;
  if (T * k > kPermSingle && (!workspace || workspace_bytes < total)) return LBMOE_ERR_WORKSPACE;
  int32_t st = check_device();
  if (st != LBMOE_OK) return st;
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (T == 0) {
    LBMOE_TRY(launch_fill_i32(counts, E, 0, s));
    LBMOE_TRY(launch_fill_i32(offsets, E + 1, 0, s));
    return LBMOE_OK;
  }
  char* ws = static_cast<char*>(workspace);
  LBMOE_TRY(launch_permute(topk_idx, idx_bytes, T, k, E, false, counts, offsets, perm_tok,
                           perm_slot, inv, ws ? reinterpret_cast<int32_t*>(ws + h) : nullptr,
                           ws ? reinterpret_cast<int32_t*>(ws + b) : nullptr,
                           ws ? reinterpret_cast<int32_t*>(ws + l) : nullptr, s));
  return LBMOE_OK;
}

int32_t lbmoe_experts(const lbmoe_layer* layer, const void* x, const void* topk_idx,
                      int32_t idx_bytes, const void* topk_w, int64_t T, void* y,
                      void* workspace, size_t workspace_bytes, void* stream) {
  int32_t st = check_shape(layer);
  if (st != LBMOE_OK) return st;
  const lbmoe_layer& L = *layer;
  if ((st = check_expert_ptrs(L)) != LBMOE_OK) return st;
  if ((st = check_T(L, T)) != LBMOE_OK) return st;
  if (idx_bytes != 4 && idx_bytes != 8) return LBMOE_ERR_DTYPE;
  if (T == 0) return LBMOE_OK;
  if (!x || !topk_idx || !topk_w || !y || !workspace) return LBMOE_ERR_NULL;
  const WsLayout w = ws_layout(L, T);
  if (workspace_bytes < w.total) return LBMOE_ERR_WORKSPACE;
  if ((st = check_device()) != LBMOE_OK) return st;
  return run_experts(L, x, topk_idx, idx_bytes, topk_w, nullptr, T, y, workspace, w, false,
                     static_cast<hipStream_t>(stream));
}

// The dense SwiGLU MLP runs as the shared-expert group of a one-expert layer; the routed
// fields only size the (unused) routed part of the workspace.
static int32_t dense_mlp_layer(int32_t H, int32_t Is, int32_t dtype, lbmoe_layer* L) {
  std::memset(L, 0, sizeof(*L));
  L->hidden_size = H;
  L->num_experts = 1;
  L->top_k = 1;
  L->moe_intermediate_size = 256;
  L->shared_intermediate_size = Is;
  L->weight_dtype = dtype;
  if (Is <= 0) return LBMOE_ERR_SHAPE;
  return check_shape(L);
}

int32_t lbmoe_dense_mlp_workspace_size(int32_t H, int32_t Is, int32_t weight_dtype, int64_t T,
                                       size_t* bytes) {
  if (!bytes) return LBMOE_ERR_NULL;
  lbmoe_layer L;
  int32_t st = dense_mlp_layer(H, Is, weight_dtype, &L);
  if (st != LBMOE_OK) return st;
  if ((st = check_T(L, T)) != LBMOE_OK) return st;
  *bytes = ws_layout(L, T).total;
  return LBMOE_OK;
}

int32_t lbmoe_dense_mlp(const void* gate_proj, const void* up_proj, const void* down_proj,
                        const float* gate_scale, const float* up_scale,
                        const float* down_scale, int32_t H, int32_t Is, int32_t weight_dtype,
                        const void* x, int64_t T, void* out, void* workspace,
                        size_t workspace_bytes, void* stream) {
  lbmoe_layer L;
  int32_t st = dense_mlp_layer(H, Is, weight_dtype, &L);
  if (st != LBMOE_OK) return st;
  L.shared_gate_proj = gate_proj;
  L.shared_up_proj = up_proj;
  L.shared_down_proj = down_proj;
  L.shared_gate_scale = gate_scale;
  L.shared_up_scale = up_scale;
  L.shared_down_scale = down_scale;
  if (!gate_proj || !up_proj || !down_proj) return LBMOE_ERR_NULL;
  if (is_fp8(L) && (!gate_scale || !up_scale || !down_scale)) return LBMOE_ERR_NULL;
  if ((st = check_T(L, T)) != LBMOE_OK) return st;
  if (T == 0) return LBMOE_OK;
  if (!x || !out || !workspace) return LBMOE_ERR_NULL;
  const WsLayout w = ws_layout(L, T);
  if (workspace_bytes < w.total) return LBMOE_ERR_WORKSPACE;
  if ((st = check_device()) != LBMOE_OK) return st;
  hipStream_t s = static_cast<hipStream_t>(stream);
  GroupWeights gw = group_weights(L, true, T);
  gw.g0 = L.num_experts;
  gw.groups = 1;
  gw.sh_row0 = 0;
  void* act = at<void>(workspace, w, R_ACT);
  const int Imax = std::max(L.moe_intermediate_size, Is);
  if (is_fp8(L)) {
    void* xq = at<void>(workspace, w, R_XQ);
    float* xs = at<float>(workspace, w, R_XS);
    void* actq = at<void>(workspace, w, R_ACTQ);
    float* acts = at<float>(workspace, w, R_ACTS);
    LBMOE_TRY(launch_quant_groups_fp8(x, T, H, H, xq, xs, s));
    LBMOE_TRY(launch_gate_up_fp8(gw, xq, xs, nullptr, nullptr, nullptr, T, 1, Imax, act, s));
    LBMOE_TRY(launch_quant_groups_fp8(act, T, Imax, Imax, actq, acts, s));
    LBMOE_TRY(launch_down_fp8(gw, actq, acts, Imax, nullptr, nullptr, T, 1, out, s));
    return LBMOE_OK;
  }
  LBMOE_TRY(launch_gate_up_bf16(gw, x, nullptr, nullptr, nullptr, T, 1, Imax, act, s));
  LBMOE_TRY(launch_down_bf16(gw, act, Imax, nullptr, nullptr, T, 1, out, s));
  return LBMOE_OK;
}

int32_t lbmoe_quantize_fp8_blocks(const void* w, int64_t batch, int32_t N, int32_t K, void* q,
                                  float* scale, void* stream) {
  if (!w || !q || !scale) return LBMOE_ERR_NULL;
  if (batch < 0 || N <= 0 || K <= 0 || N % 128 != 0 || K % 128 != 0) return LBMOE_ERR_SHAPE;
  if (batch == 0) return LBMOE_OK;
  int32_t st = check_device();
  if (st != LBMOE_OK) return st;
  LBMOE_TRY(launch_quant_blocks_fp8(w, batch, N, K, q, scale, static_cast<hipStream_t>(stream)));
  return LBMOE_OK;
}

}  // extern "C"
