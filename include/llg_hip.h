/*
 * llg_hip.h -- C ABI of the MI355X (gfx950) sparse-FFN library.
 *
 * Drop-in replacement for the reference's native bridge
 * metal/metal_bridge.h:1-20 (AndersHsueh/llama.go), extended with the
 * sparse-FFN hot path that the reference runs on the CPU:
 *   predictor + selection   inference/predictor.go:51-83
 *   gathered sparse FFN     inference/ffn_flash.go:254-299
 *   dense dequant FFN       inference/forward.go:318-353, tensor/ops.go:39-60
 *   sliding window          inference/window.go:71-180
 *   MoE router + experts    inference/moe_forward.go:32-150
 *   GGUF dequant            tensor/dtype.go:12-82, 249-293, 417-443
 *
 * Conventions (kept from metal_bridge.h):
 *   - an opaque device handle; llg_hip_init returns NULL when no GPU is usable;
 *   - every entry point returns int: 0 = OK, <0 = argument error (LLG_E_*),
 *     >0 = a hipError_t from the runtime;  llg_hip_last_error() describes it;
 *   - llg_hip_* entry points take caller-owned HOST buffers and are synchronous
 *     (they return after the device work has completed, like the Metal
 *     bridge's commit + waitUntilCompleted);
 *   - llg_hipd_* entry points take DEVICE pointers for activations/outputs,
 *     enqueue on the handle's stream and return without waiting; call
 *     llg_hip_sync() (or order work on llg_hip_stream()) before reading results;
 *   - weights are uploaded once into library-owned device objects identified
 *     by int64 handles (cgo forbids C from keeping Go pointers after a call);
 *   - a handle is not thread-safe: callers serialise calls per handle.
 *
 * Element types are GGUF ggml_type codes (gguf/types.go:40-61): F32=0, F16=1,
 * Q4_0=2, Q8_0=8.  Activations are model.ActivationType (model/model.go:97-103):
 * ReLU=0, GELU=1, SiLU=2.
 */
#ifndef LLG_HIP_H
#define LLG_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef void *LlgHipDevice;

enum {
    LLG_TYPE_F32 = 0,
    LLG_TYPE_F16 = 1,
    LLG_TYPE_Q4_0 = 2,
    LLG_TYPE_Q8_0 = 8,
};

/* model.ActivationType (model.go:97-103).  Every `act` argument takes one of
 * these; any other value is LLG_E_ARG. */
enum { LLG_ACT_RELU = 0, LLG_ACT_GELU = 1, LLG_ACT_SILU = 2 };

enum {
    LLG_OK = 0,
    LLG_E_ARG = -1,     /* null pointer, non-positive or mismatched size */
    LLG_E_TYPE = -2,    /* ggml type not supported (dtype.go:266) */
    LLG_E_ALIGN = -3,   /* element count not a multiple of the block size (types.go:98-100) */
    LLG_E_RANGE = -4,   /* neuron / row index out of range (storage.go:292-294) */
    LLG_E_HANDLE = -5,  /* unknown or wrong-kind object handle */
    LLG_E_NOMEM = -6,   /* device or pinned allocation failed */
    LLG_E_HPARAM = -7,  /* invalid MoE hparams (moe_forward.go:38-40) */
    LLG_E_NODEV = -8,   /* null device handle */
    LLG_E_SCRATCH = -9, /* workload needs more than the fixed scratch of the
                           allocation-free entry points */
};

/* ---- device lifecycle: metal_bridge.h:7-10 ------------------------------ */
int llg_hip_available(void);                  /* llama_metal_available */
LlgHipDevice llg_hip_init(void);              /* llama_metal_init: NULL if unavailable */
void llg_hip_free(LlgHipDevice dev);          /* llama_metal_free */
const char *llg_hip_last_error(LlgHipDevice dev);
/* The hipStream_t (as void*) that llg_hipd_* calls enqueue on. */
void *llg_hip_stream(LlgHipDevice dev);
int llg_hip_sync(LlgHipDevice dev);
/* Bytes of the handle's growable device workspace (0 until an entry point
 * first needs one; it only grows, until llg_hip_free).  No counterpart in the
 * reference: a diagnostic that lets a caller confirm that the
 * allocation-free entry points left the workspace untouched. */
int llg_hip_workspace_bytes(LlgHipDevice dev, size_t *bytes);

/* ---- Metal-parity entry points: metal_bridge.h:12-20 -------------------- */
/* y[rows] = W[rows*cols] @ x[cols], fp32 (llama_metal_matvec, used by
 * inference/forward.go:395-405). */
int llg_hip_matvec(LlgHipDevice dev, const float *w, int rows, int cols, const float *x,
                   float *y);
/* out[n] = x[n] / sqrt(sum(x^2)/n + eps) * weight[n] (llama_metal_rmsnorm,
 * used by inference/forward.go:409-418). */
int llg_hip_rmsnorm(LlgHipDevice dev, const float *x, const float *weight, float *out, int n,
                    float eps);

/* ---- weight residency (replaces flash/storage.go reads: weights live in HBM) */
/* A row-major matrix of `rows` rows x `cols` elements, given as GGUF tensor
 * bytes (rows * ByteSize(cols), gguf/types.go:90-102).  Row r is addressed as
 * in flash/storage.go:296 (offset = r * ByteSize(cols)).  *mat gets a handle. */
int llg_hip_upload_matrix(LlgHipDevice dev, const void *gguf_raw, int ggml_type, int rows,
                          int cols, int64_t *mat);
/* Same, from a device pointer to the GGUF bytes (copied; source not retained). */
int llg_hipd_upload_matrix(LlgHipDevice dev, const void *d_gguf_raw, int ggml_type, int rows,
                           int cols, int64_t *mat);
/* Row-column bundle (flash/bundle.go:37-111): neuron i stores ffn_up row i
 * (up_raw, ff rows of ByteSize(h)) contiguous with ffn_down row i (down_t_raw,
 * the [ff x h] layout the sparse path reads, ffn_flash.go:267).  Bytes stay
 * quantized; one contiguous span per neuron. */
int llg_hip_upload_bundle(LlgHipDevice dev, const void *up_raw, const void *down_t_raw,
                          int ggml_type, int h, int ff, int64_t *bundle);
int llg_hipd_upload_bundle(LlgHipDevice dev, const void *d_up_raw, const void *d_down_t_raw,
                           int ggml_type, int h, int ff, int64_t *bundle);
/* Retires a handle (LLG_E_HANDLE if unknown or already retired).  An object
 * that a window or model still reads (a window's bundle, a model's weights)
 * stays in device memory until the last of those is released; any other
 * object is freed now.  llg_hip_free frees everything. */
int llg_hip_release(LlgHipDevice dev, int64_t handle);
/* Per-neuron byte stride of a bundle and per-row stride of a matrix in HBM. */
int llg_hip_object_info(LlgHipDevice dev, int64_t handle, int *ggml_type, int *rows,
                        int *cols, int64_t *row_stride);

/* ---- dequant: tensor/dtype.go:12-82 (bit-exact with float16ToFloat32 :417-443) */
/* Rows [row0, row0+nrows) of a matrix (or, for a bundle, neuron rows with the
 * up row first then the down row: 2*h floats per neuron) to fp32. */
int llg_hip_dequant(LlgHipDevice dev, int64_t handle, int row0, int nrows, float *out);

/* ---- predictor: inference/predictor.go:51-83 ---------------------------- */
/* wup: F32 matrix [rank x h]; wout: F32 matrix [ff x rank]; bias: F32 [1 x ff]
 * matrix or 0.  a: the predictor input [h] (the layer's attention output).
 * active (capacity ff) receives {i : logit_i > threshold} ascending;
 * logits (optional, [ff]) receives the logits. */
int llg_hip_predict(LlgHipDevice dev, int64_t wup, int64_t wout, int64_t bias, const float *a,
                    float threshold, int32_t *active, int *n_active, float *logits);
/* Selection alone on given logits (predictor.go:76-82): the bit-exact hook. */
int llg_hip_select(LlgHipDevice dev, const float *logits, int ff, float threshold,
                   int32_t *active, int *n_active);

/* ---- sparse FFN: inference/ffn_flash.go:254-299 ------------------------- */
/* out[h] = sum_{j in active} act(up_j . x) * down_j, skipping zero activations;
 * n_active == 0 gives zeros.  Indices must be in [0, ff). */
int llg_hip_ffn_sparse(LlgHipDevice dev, int64_t bundle, const float *x, const int32_t *active,
                       int n_active, int act, float *out);
/* Path 2 of ffnFlash (ffn_flash.go:225-231): predict on `a`, then sparse FFN
 * on `x`, without a host round trip.  active/n_active optional outputs. */
int llg_hip_ffn_predict_sparse(LlgHipDevice dev, int64_t wup, int64_t wout, int64_t bias,
                               int64_t bundle, const float *a, const float *x, float threshold,
                               int act, float *out, int32_t *active, int *n_active);

/* ---- dense path: inference/forward.go:318-353, tensor/ops.go:39-60 ------- */
/* y[rows] = dequant(W) @ x for any supported matrix type. */
int llg_hip_matvec_q(LlgHipDevice dev, int64_t mat, const float *x, float *y);
/* out = down @ act(up @ x); up [ff x h], down [h x ff] (standard GGUF layout). */
int llg_hip_ffn_dense(LlgHipDevice dev, int64_t up, int64_t down, const float *x, int act,
                      float *out);
/* ffnSwiGLU (forward.go:368-389), the dense path of SiLU models (forward.go:
 * 328-329): out = down @ (silu(gate @ x) * (up @ x)); gate and up [ff x h] of
 * one type, down [h x ff]. */
int llg_hip_ffn_swiglu(LlgHipDevice dev, int64_t gate, int64_t up, int64_t down, const float *x,
                       float *out);

/* ---- sliding window: inference/window.go -------------------------------- */
/* NewNeuronCache (window.go:48-63) over a bundle, window size k >= 1. */
int llg_hip_window_create(LlgHipDevice dev, int64_t bundle, int k, int64_t *win);
/* Update (window.go:71-117): evict neurons only the expiring slot needed,
 * gather-copy the active neurons not resident, record the set.  n_loaded
 * receives |toLoad|, n_resident NumCached() (window.go:183); both optional. */
int llg_hip_window_update(LlgHipDevice dev, int64_t win, const int32_t *active, int n_active,
                          int *n_loaded, int *n_resident);
/* FFNForward (window.go:143-180) over the resident rows. */
int llg_hip_window_ffn(LlgHipDevice dev, int64_t win, const float *x, const int32_t *active,
                       int n_active, int act, float *out);
/* Resident flags: resident[n] = 1 if neuron n is resident (capacity ff). */
int llg_hip_window_resident(LlgHipDevice dev, int64_t win, uint8_t *resident, int *n_resident);

/* ---- MoE: inference/moe_forward.go:32-150 ------------------------------- */
/* router: F32 matrix [n_exp x hidden]; gate_exps/up_exps: matrices of
 * n_exp*eff rows x hidden (GGUF dims [hidden, eff, n_exp]); down_exps:
 * n_exp*hidden rows x eff (dims [eff, hidden, n_exp]).  x: [n_tok x hidden];
 * out: [n_tok x hidden].  ids/weights (optional, [n_tok x k]) receive the
 * chosen experts in accumulation order (descending probability, ties to the
 * lower index) and p/wsum.  Batches of n_tok >= 16 Q4_0 tokens with hidden a
 * multiple of 256 and expert width a multiple of 128 are grouped per expert
 * and run as grouped MFMA GEMMs (f16 operands, fp32 accumulation); other
 * batches run the per-token decode kernels. */
int llg_hip_moe_ffn(LlgHipDevice dev, int64_t router, int64_t gate_exps, int64_t up_exps,
                    int64_t down_exps, int n_exp, int k, const float *x, int n_tok, float *out,
                    int32_t *ids, float *weights);
/* Router stage on given logits [n_tok x n_exp] (softmax, top-k, renorm). */
int llg_hip_moe_route(LlgHipDevice dev, const float *logits, int n_tok, int n_exp, int k,
                      int32_t *ids, float *weights);

/* ---- Falcon-architecture decode around the sparse FFN ------------------- */
/* ForwardFlash (inference/ffn_flash.go:115-185) on the Falcon parallel layout
 * with ffnFlash path 2, attention as forward.go:206-310 (no biases, RoPE with
 * rope_base, MQA/GQA), KV cache as kvcache/kvcache.go:25-82, greedy argmax as
 * cmd/generate.go:197-205.  dims = {n_layers, hidden, n_heads, n_kv_heads,
 * head_dim (64 or 128), ff, vocab, max_seq}.  layer_handles holds 7 handles
 * per layer: attn_norm weight, attn_norm bias (F32 [1 x hidden]), wqkv (the
 * rows of Wq, Wk, Wv stacked), wo, predictor WUp, predictor WOut (F32), the
 * FFN bundle.  thresholds: one per layer.  The model owns its KV cache
 * (n_layers x max_seq x 2 x n_kv_heads x head_dim floats); the token at
 * position pos is written to cache row pos (the reference commits after
 * every token, generate.go:94,119). */
int llg_hip_falcon_create(LlgHipDevice dev, const int32_t *dims, float rope_base,
                          float norm_eps, int act, int64_t embed,
                          const int64_t *layer_handles, const float *thresholds,
                          int64_t out_norm_w, int64_t out_norm_b, int64_t lm_head,
                          int64_t *model);
int llg_hip_falcon_set_thresholds(LlgHipDevice dev, int64_t model, const float *thresholds);
/* One token (ForwardFlash(token, pos)); logits [vocab], next_token (greedy)
 * and n_active [n_layers] are optional host outputs.  pred_logits (optional,
 * [n_layers x ff]) receives every layer's predictor logits (predictor.go:57-73)
 * from an extra predict-only pass, for calibrating the thresholds. */
int llg_hip_falcon_forward(LlgHipDevice dev, int64_t model, int32_t token, int pos,
                           float *logits, int32_t *next_token, int32_t *n_active,
                           float *pred_logits);

/* ---- device-pointer (async) variants for HBM-resident callers ----------- */
int llg_hipd_predict(LlgHipDevice dev, int64_t wup, int64_t wout, int64_t bias,
                     const float *d_a, float threshold, int32_t *d_active,
                     int32_t *d_n_active, float *d_logits);
/* n_active is read on the device from d_n_active; d_active must hold that
 * many entries.  Indices are not checked on the host on this path (they come
 * from llg_hipd_predict or a checked caller); the kernels clamp the count to
 * ff and treat an index outside [0, ff) as an inactive neuron, so such a list
 * gives meaningless results but no out-of-bounds access.  The same holds for
 * llg_hipd_window_step, whose window state such a list leaves meaningless. */
int llg_hipd_ffn_sparse(LlgHipDevice dev, int64_t bundle, const float *d_x,
                        const int32_t *d_active, const int32_t *d_n_active, int act,
                        float *d_out);
int llg_hipd_ffn_predict_sparse(LlgHipDevice dev, int64_t wup, int64_t wout, int64_t bias,
                                int64_t bundle, const float *d_a, const float *d_x,
                                float threshold, int act, float *d_out, int32_t *d_active,
                                int32_t *d_n_active);
/* Allocation-free form of llg_hipd_ffn_predict_sparse: no counterpart in the
 * reference.  It is for callers that cannot allocate device memory (code under
 * HIP graph capture, tight serving loops, harnesses that forbid hipMalloc).
 * Same arguments, results and errors; its kernels take their sync area (the
 * hand-off of the predictor's hidden units, zero at load and never cleared),
 * tile masks and partial output rows from a fixed array in each GPU's memory
 * (8 MiB per GPU, held until the process ends) instead of the handle's
 * growable workspace, and it calls no hipMalloc, hipFree or hipMemset.  A
 * predictor and bundle whose workspace exceeds the array give LLG_E_SCRATCH
 * (the Falcon-7B layer, rank 128 x d_ff 18176, needs 5.0 MiB).  Every call on one GPU shares
 * the array: calls that overlap on one GPU (from several handles or streams)
 * race; calls ordered on one stream do not. */
int llg_hipd_ffn_predict_sparse_noalloc(LlgHipDevice dev, int64_t wup, int64_t wout,
                                        int64_t bias, int64_t bundle, const float *d_a,
                                        const float *d_x, float threshold, int act,
                                        float *d_out, int32_t *d_active,
                                        int32_t *d_n_active);
int llg_hipd_matvec_q(LlgHipDevice dev, int64_t mat, const float *d_x, float *d_y);
int llg_hipd_ffn_dense(LlgHipDevice dev, int64_t up, int64_t down, const float *d_x, int act,
                       float *d_out);
int llg_hipd_ffn_swiglu(LlgHipDevice dev, int64_t gate, int64_t up, int64_t down,
                        const float *d_x, float *d_out);
int llg_hipd_window_step(LlgHipDevice dev, int64_t win, const float *d_x,
                         const int32_t *d_active, const int32_t *d_n_active, int act,
                         float *d_out);
int llg_hipd_moe_ffn(LlgHipDevice dev, int64_t router, int64_t gate_exps, int64_t up_exps,
                     int64_t down_exps, int n_exp, int k, const float *d_x, int n_tok,
                     float *d_out, int32_t *d_ids, float *d_weights);
/* One token of the Falcon model on the stream: embeds *d_token (device int32),
 * writes the greedy next token to *d_next_token (may equal d_token) and, if
 * d_logits is given, the logits.  A decode loop chains calls without waiting. */
int llg_hipd_falcon_step(LlgHipDevice dev, int64_t model, const int32_t *d_token, int pos,
                         int32_t *d_next_token, float *d_logits);

#ifdef __cplusplus
}
#endif
#endif /* LLG_HIP_H */
