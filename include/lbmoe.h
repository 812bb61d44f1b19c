/*
 * lbmoe.h - C ABI of the MI355X (gfx950) sparse-MoE feed-forward layer.
 *
 * The layer is the reference's Qwen3_5SparseMoeBlock (nanovllm/models/qwen3_5.py:881-905):
 *   y = sum_s w[t,s] * down_e(silu(gate_e x) * up_e x)  +  sigmoid(x.w_sg) * shared(x)
 * with (w, e) = top-k of softmax(bf16(x . Wg^T)) renormalised.
 *
 * Conventions
 *  - All pointers are device pointers unless stated; tensors are row-major, last dim
 *    contiguous, with the reference's parameter layouts (qwen3_5.py:765, :795-800,
 *    :912-914, :897).
 *  - `stream` is a hipStream_t passed as void* (NULL = the null stream). Every entry
 *    point only enqueues work on that stream: no host synchronisation, no device
 *    allocation, grids that depend on T and the layer shape only. The entry points are
 *    therefore safe inside HIP graph capture and on any caller-chosen stream.
 *  - Scratch memory is caller-owned: size it with lbmoe_workspace_size and pass it in.
 *  - Every entry point returns an lbmoe_status; a negative value means nothing was
 *    enqueued (argument errors) or the launch failed. There is no fallback path.
 *  - The library's only global state is set once per device and then read: the
 *    architecture check, the device's CU count and the address of lbmoe_forward_static's
 *    workspace. Concurrent calls on different streams with different workspaces are
 *    independent; lbmoe_forward_static calls on one device share one workspace (see there).
 */
#ifndef LBMOE_H
#define LBMOE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define LBMOE_ABI_VERSION 2

typedef enum lbmoe_status {
  LBMOE_OK = 0,
  LBMOE_ERR_NULL = -1,        /* a required pointer is NULL                         */
  LBMOE_ERR_SHAPE = -2,       /* unsupported or inconsistent sizes                  */
  LBMOE_ERR_DTYPE = -3,       /* unknown weight dtype / index width                 */
  LBMOE_ERR_WORKSPACE = -4,   /* workspace smaller than lbmoe_workspace_size        */
  LBMOE_ERR_DEVICE = -5,      /* current device is not gfx950 / no device           */
  LBMOE_ERR_LAUNCH = -6,      /* a kernel launch reported an error                  */
  LBMOE_ERR_STATIC_LIMIT = -7 /* lbmoe_forward_static: the call needs more workspace than
                                 LBMOE_STATIC_WORKSPACE_BYTES                          */
} lbmoe_status;

typedef enum lbmoe_weight_dtype {
  LBMOE_W_BF16 = 0,           /* expert weights bf16                                */
  LBMOE_W_FP8_E4M3 = 1        /* expert weights OCP e4m3fn + fp32 128x128 block scales */
} lbmoe_weight_dtype;

/*
 * One MoE layer: shapes plus borrowed device pointers to its parameters.
 * Shapes are the reference config's MoE fields (nanovllm/config.py:98-102).
 * Parameter names in the comments are the reference module's (qwen3_5.py:881-917).
 */
typedef struct lbmoe_layer {
  int32_t hidden_size;              /* H  (multiple of 128)                              */
  int32_t num_experts;              /* E  (1..1024)                                      */
  int32_t top_k;                    /* k  (1..min(E,32))                                 */
  int32_t moe_intermediate_size;    /* I  (multiple of 128)                              */
  int32_t shared_intermediate_size; /* Is (0 = no shared expert, else multiple of 128)   */
  int32_t weight_dtype;             /* lbmoe_weight_dtype                                */
  const void*  gate_weight;         /* gate.weight            bf16 [E,H]                 */
  const float* logit_bias;          /* optional fp32 [E] added to the upcast logits      */
  const void*  gate_up_proj;        /* experts.gate_up_proj   [E,2I,H] (gate rows first) */
  const void*  down_proj;           /* experts.down_proj      [E,H,I]                    */
  const float* gate_up_scale;       /* fp8 only: fp32 [E,2I/128,H/128]                   */
  const float* down_scale;          /* fp8 only: fp32 [E,H/128,I/128]                    */
  const void*  shared_gate_proj;    /* shared_expert.gate_proj.weight [Is,H]             */
  const void*  shared_up_proj;      /* shared_expert.up_proj.weight   [Is,H]             */
  const void*  shared_down_proj;    /* shared_expert.down_proj.weight [H,Is]             */
  const void*  shared_expert_gate;  /* shared_expert_gate.weight bf16 [1,H]              */
  const float* shared_gate_scale;   /* fp8 only: fp32 [Is/128,H/128]                     */
  const float* shared_up_scale;     /* fp8 only: fp32 [Is/128,H/128]                     */
  const float* shared_down_scale;   /* fp8 only: fp32 [H/128,Is/128]                     */
  /* Optional, bf16 layers only (NULL: not used): copies of the expert weights in the tiled
   * layout that lbmoe_pack_weights writes. Each one that is set replaces its checkpoint tensor
   * in the prefill-sized GEMMs, which stream it markedly faster; the checkpoint tensors stay
   * required (decode-sized batches read them). No counterpart in the reference: the module's
   * parameters are the checkpoint tensors, and these are derived from them once. */
  const void*  gate_up_tiled;        /* from gate_up_proj, same bytes                     */
  const void*  down_tiled;           /* from down_proj, same bytes                        */
  const void*  shared_gate_up_tiled; /* from shared gate_proj + up_proj, 2*Is*H bf16      */
  const void*  shared_down_tiled;    /* from shared down_proj, same bytes                 */
} lbmoe_layer;

/* Human-readable name of a status code (static string). */
const char* lbmoe_status_string(int32_t status);

/* LBMOE_ABI_VERSION of the loaded library. */
int32_t lbmoe_abi_version(void);

/* Host-side validation of shapes, dtype and required pointers. No device access. */
int32_t lbmoe_check_layer(const lbmoe_layer* layer);

/* Workspace bytes needed by lbmoe_forward / lbmoe_experts for T tokens. Pure host
 * arithmetic; checks shapes and dtype only. */
int32_t lbmoe_workspace_size(const lbmoe_layer* layer, int64_t T, size_t* bytes);

/* Byte range of one named region inside the workspace of a T-token call, for
 * inspection of intermediates after lbmoe_forward. region: 0 logits bf16 [T,E],
 * 1 topk_idx int32 [T,k], 2 topk_w bf16 [T,k], 3 shared_gate fp32 [T],
 * 4 counts int32 [E+1], 5 offsets int32 [E+2], 6 perm_tok int32 [T*k+T],
 * 7 perm_slot int32 [T*k], 8 inv int32 [T,k], 9 act bf16 [T*k+T, max(I,Is)]
 * (not written by the fp8 prefill path, whose gate_up stores the quantised act directly),
 * 10 expert_out bf16 [T*k+T, H] (not written for bf16 batches of at most 4 tokens, whose
 * down projection and combine run as one kernel), 11 xn bf16 [T,H] (the block input
 * lbmoe_forward_norm computes). */
int32_t lbmoe_workspace_region(const lbmoe_layer* layer, int64_t T, int32_t region,
                               size_t* offset, size_t* bytes);

/*
 * The whole block: Qwen3_5SparseMoeBlock.forward (qwen3_5.py:899-905).
 * x bf16 [T,H] -> y bf16 [T,H]. T >= 0 (T = 0 enqueues nothing).
 */
int32_t lbmoe_forward(const lbmoe_layer* layer, const void* x, int64_t T, void* y,
                      void* workspace, size_t workspace_bytes, void* stream);

/*
 * The decoder layer's MLP half: qwen3_5.py:998-1004. hidden (the attention output) and
 * residual are bf16 [T,H]; h = residual + hidden (bf16) is written to residual_out, and the
 * block runs on x = Qwen3_5RMSNorm(h) (qwen3_5.py:39-55: fp32 h / sqrt(mean(h^2) + eps), times
 * (1 + norm_weight), rounded to bf16; norm_weight bf16 [H]) into y bf16 [T,H]. For decode-sized
 * T the add and the norm run inside the router kernel. residual_out must not overlap
 * residual or hidden; x is kept in the workspace's xn region.
 */
int32_t lbmoe_forward_norm(const lbmoe_layer* layer, const void* hidden, const void* residual,
                           const void* norm_weight, float eps, int64_t T, void* y,
                           void* residual_out, void* workspace, size_t workspace_bytes,
                           void* stream);

/*
 * Writes the tiled copies of a bf16 layer's expert weights (the lbmoe_layer *_tiled fields)
 * from its checkpoint tensors: gate_up_tiled and down_tiled (as many bytes as gate_up_proj and
 * down_proj), and, with a shared expert, shared_gate_up_tiled (2*Is*H bf16) and
 * shared_down_tiled (H*Is bf16). Run once after the weights are loaded (or changed); the copies
 * are device memory the caller owns and must not overlap the checkpoint tensors. Shapes the
 * prefill GEMMs do not tile (H not a multiple of 256) return LBMOE_ERR_SHAPE, fp8 layers
 * LBMOE_ERR_DTYPE. No counterpart in the reference (a load-time layout step, like the fp8
 * quantisation of lbmoe_quantize_fp8_blocks).
 */
int32_t lbmoe_pack_weights(const lbmoe_layer* layer, void* gate_up_tiled, void* down_tiled,
                           void* shared_gate_up_tiled, void* shared_down_tiled, void* stream);

/* Bytes of the device workspace lbmoe_forward_static uses: one array per GPU, part of the
 * library's device code, so every GPU that runs any of the library's kernels holds it until the
 * process ends, whether or not lbmoe_forward_static is called. */
#define LBMOE_STATIC_WORKSPACE_BYTES (64u << 20)

/*
 * lbmoe_forward without a workspace argument, for callers that cannot allocate device memory
 * (code under HIP graph capture, tight serving loops, harnesses that forbid hipMalloc). No
 * counterpart in the reference. The workspace is a library-owned device array of
 * LBMOE_STATIC_WORKSPACE_BYTES per GPU; calls needing more (lbmoe_workspace_size of the
 * layer at T) return LBMOE_ERR_STATIC_LIMIT and enqueue nothing. The call allocates nothing
 * (no hipMalloc, no hipFree). Every call on one GPU uses the same array: calls that overlap on
 * one GPU (different streams, different host threads) race, and the array keeps the last
 * call's intermediates (nothing in it needs to start at zero). Results are those of
 * lbmoe_forward, bit for bit.
 */
int32_t lbmoe_forward_static(const lbmoe_layer* layer, const void* x, int64_t T, void* y,
                             void* stream);

/* Number of events lbmoe_forward_profiled records. */
#define LBMOE_PROFILE_EVENTS 7

/*
 * lbmoe_forward with stage timing (instrumentation; no counterpart in the reference).
 * events[0..6] are caller-created hipEvent_t handles (passed as void*), recorded on `stream`
 * before the first kernel and after each stage: router logits, top-k routing, permutation,
 * gate_up + SiLU*mul, down projection, combine. hipEventElapsedTime between consecutive
 * events gives each stage's device time. Batches that lbmoe_forward routes and permutes in one
 * kernel (up to 16 tokens for at most 128 experts, else up to 4) run it here too: its time is
 * the routing stage's, and the permutation stage is empty. bf16 batches of at most 4 tokens
 * with T*top_k <= 64 route and permute inside the gate_up kernel: both of those stages are
 * empty and the gate_up stage includes them. bf16 batches of at most 4 tokens run the down
 * projection and the combine as one kernel, timed as the down stage (the combine stage is
 * empty). bf16 decode batches of at most 256 tokens with T*top_k >= E permute inside the
 * gate_up kernel: the permutation stage is empty. Prefill batches (from 1024 tokens, with
 * the LDS-tiled expert GEMMs) of at most 128 experts and top_k <= 16 select the experts inside
 * the router kernel: the routing stage is empty, and the permutation stage also builds the
 * GEMMs' tile list (otherwise launched with gate_up).
 */
int32_t lbmoe_forward_profiled(const lbmoe_layer* layer, const void* x, int64_t T, void* y,
                               void* workspace, size_t workspace_bytes, void* stream,
                               void* const* events, int32_t n_events);

/*
 * Router logits: the F.linear of Qwen3_5TopKRouter.forward (qwen3_5.py:769).
 * x bf16 [T,H] -> logits bf16 [T,E] (fp32 accumulation, round-to-nearest-even).
 */
int32_t lbmoe_router_logits(const lbmoe_layer* layer, const void* x, int64_t T,
                            void* logits, void* stream);

/*
 * Routing from logits: softmax, top-k, renormalise, bf16 cast of
 * Qwen3_5TopKRouter.forward (qwen3_5.py:770-774), plus the optional logit bias.
 * logits bf16 [T,E] -> topk_idx [T,k] (idx_bytes 4: int32, 8: int64), topk_w bf16 [T,k].
 * Order within a row: descending (logit + bias), ties by ascending expert index.
 * When x and the layer's shared_expert_gate are non-NULL and shared_gate is non-NULL,
 * also writes shared_gate[t] = sigmoid(bf16(x[t] . w_sg)) as fp32 (qwen3_5.py:903).
 */
int32_t lbmoe_route(const lbmoe_layer* layer, const void* logits, const void* x, int64_t T,
                    void* topk_idx, int32_t idx_bytes, void* topk_w, float* shared_gate,
                    void* stream);

/* Workspace bytes of lbmoe_permute. */
int32_t lbmoe_permute_workspace_size(int64_t T, int32_t k, int32_t E, size_t* bytes);

/*
 * Expert sort of the (token, slot) pairs: _forward_sparse's one_hot / nonzero / where
 * (qwen3_5.py:823-833), as explicit arrays ordered by the key (expert, slot, token).
 * topk_idx [T,k] (idx_bytes 4 or 8, values in [0,E)) -> counts int32 [E],
 * offsets int32 [E+1] (exclusive scan), perm_tok / perm_slot int32 [T*k],
 * inv int32 [T,k] with perm_*[inv[t,s]] == (t,s).
 */
int32_t lbmoe_permute(const void* topk_idx, int32_t idx_bytes, int64_t T, int32_t k,
                      int32_t E, int32_t* counts, int32_t* offsets, int32_t* perm_tok,
                      int32_t* perm_slot, int32_t* inv, void* workspace,
                      size_t workspace_bytes, void* stream);

/*
 * Routed experts only: Qwen3_5Experts.forward(x, idx, w) (qwen3_5.py:802-874).
 * x bf16 [T,H], topk_idx [T,k] (idx_bytes 4 or 8), topk_w bf16 [T,k] -> y bf16 [T,H].
 */
int32_t lbmoe_experts(const lbmoe_layer* layer, const void* x, const void* topk_idx,
                      int32_t idx_bytes, const void* topk_w, int64_t T, void* y,
                      void* workspace, size_t workspace_bytes, void* stream);

/* Workspace bytes of lbmoe_dense_mlp for T tokens. */
int32_t lbmoe_dense_mlp_workspace_size(int32_t H, int32_t Is, int32_t weight_dtype, int64_t T,
                                       size_t* bytes);

/*
 * Dense SwiGLU MLP: Qwen3_5SharedExpertMLP.forward (qwen3_5.py:916-917), i.e. the shared
 * expert without its sigmoid gate: out = down(silu(gate_proj x) * up_proj x).
 * gate_proj / up_proj [Is,H], down_proj [H,Is] (bf16, or e4m3 with the fp32 block scales
 * [Is/128,H/128], [Is/128,H/128], [H/128,Is/128]); x bf16 [T,H] -> out bf16 [T,H].
 */
int32_t lbmoe_dense_mlp(const void* gate_proj, const void* up_proj, const void* down_proj,
                        const float* gate_scale, const float* up_scale,
                        const float* down_scale, int32_t H, int32_t Is, int32_t weight_dtype,
                        const void* x, int64_t T, void* out, void* workspace,
                        size_t workspace_bytes, void* stream);

/*
 * Offline weight conversion for LBMOE_W_FP8_E4M3 (no counterpart in the reference,
 * which has no fp8 path): w bf16 [batch,N,K] (N, K multiples of 128) ->
 * q e4m3fn [batch,N,K], scale fp32 [batch,N/128,K/128], scale = blockmax|w|/448,
 * q = e4m3(w/scale) round-to-nearest-even, saturating.
 */
int32_t lbmoe_quantize_fp8_blocks(const void* w, int64_t batch, int32_t N, int32_t K,
                                  void* q, float* scale, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* LBMOE_H */
