/*
 * refcpu.h -- CPU oracle: a plain-C restatement of llama.go's sparse-FFN
 * path (AndersHsueh/llama.go), used ONLY as the reference result by tests/, the smoke
 * check and bench.py's cpu_baseline leg.  It is never linked into, loaded by
 * or called from the product library.
 *
 * Arithmetic contract (matches the reference's Go code on amd64):
 *   - fp32 sequential accumulation in the reference's loop order, sums start at 0;
 *   - compiled with -O2 -ffp-contract=off and no fast-math (no FMA contraction);
 *   - exp/tanh evaluated in double and rounded to float where Go uses math.Exp/Tanh;
 *   - strict '>' threshold, ascending active lists;
 *   - the reference's interleaved Q4_0 nibble order and its f16->f32 conversion.
 *
 * Every function cites the reference file:line it restates.
 */
#ifndef LLG_REFCPU_H
#define LLG_REFCPU_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* GGML type codes: gguf/types.go:40-61 */
enum {
    REFCPU_F32 = 0,
    REFCPU_F16 = 1,
    REFCPU_Q4_0 = 2,
    REFCPU_Q8_0 = 8,
};

/* model.ActivationType: model/model.go:97-103 (iota order) */
enum { REFCPU_ACT_RELU = 0, REFCPU_ACT_GELU = 1, REFCPU_ACT_SILU = 2 };

/* gguf/types.go:70-102 -- bytes for n elements; -1 if the type is unknown or
 * n is not a multiple of the block size. */
int64_t refcpu_byte_size(int ggml_type, int64_t n);

/* tensor/dtype.go:417-443 */
float refcpu_f16_to_f32(uint16_t h);

/* tensor/dtype.go:249-268 (Dequantize) for F32/F16/Q8_0/Q4_0.
 * Returns the element count written, or -1 on error (bad length / type). */
int64_t refcpu_dequantize(const uint8_t *raw, int64_t nbytes, int ggml_type, float *out);

/* tensor/ops.go:39-60 -- y[i] = sum_j w[i*in+j]*x[j], sequential j. */
void refcpu_matmulvec(const float *w, int out_dim, int in_dim, const float *x, float *y);
/* Row threads of refcpu_matmulvec (default 1); results are identical for any n. */
void refcpu_set_threads(int n);

/* tensor/ops.go:168-189 and inference/ffn_flash.go:303-312 */
void refcpu_relu(float *x, int n);
void refcpu_silu(float *x, int n);
void refcpu_gelu(float *x, int n);
void refcpu_activation(int act, float *x, int n);

/* tensor/ops.go:114-135 and :138-165 */
void refcpu_rmsnorm(const float *x, const float *w, float *out, int n, float eps);
void refcpu_layernorm(const float *x, const float *w, const float *b, float *out, int n, float eps);

/* inference/forward.go:463-479 */
void refcpu_softmax_inplace(float *v, int n);

/* inference/predictor.go:76-82 -- ascending {i : logits[i] > thr}; returns count. */
int refcpu_select(const float *logits, int ff, float threshold, int32_t *active);

/* inference/predictor.go:51-83.  wup [rank x h], wout [ff x rank], bias [ff] or NULL.
 * logits_out (optional, [ff]).  Returns n_active, or -1 if weights are NULL
 * (predictor.go:52-54). */
int refcpu_predict(const float *wup, const float *wout, const float *bias, int h, int rank,
                   int ff, const float *a, float threshold, int32_t *active, float *logits_out);

/* flash/storage.go:246-319 (row addressing + per-row dequant), in memory and
 * single-threaded.  tensor_raw holds out_dim rows of ByteSize(in_dim) bytes.
 * Returns 0, or -1 on a bad type/length, -2 on an out-of-range row. */
int refcpu_read_rows(const uint8_t *tensor_raw, int ggml_type, int in_dim, int out_dim,
                     const int32_t *rows, int n_rows, float *out);

/* flash/storage.go:246-319 ReadRowsParallel: the rows of the tensor at byte
 * offset tensor_offset of the file at path, read with pread by nthreads
 * threads (32 when nthreads <= 0) pulling rows from a shared queue; each
 * thread opens its own descriptor, reads a row into a buffer of its own and
 * dequantizes it into out.  Returns 0, or the first failing row's error:
 * -1 bad type/length, -2 row out of range, -3 open failed, -4 short read. */
int refcpu_read_rows_file(const char *path, int64_t tensor_offset, int ggml_type, int in_dim,
                          int out_dim, const int32_t *rows, int n_rows, int nthreads,
                          float *out);

/* inference/ffn_flash.go:254-299.  up_raw: ffn_up, F rows of ByteSize(h).
 * down_t_raw: ffn_down stored [F rows x h] (GGUF dims [h, F]).  Returns 0 or <0. */
int refcpu_ffn_sparse_load(const uint8_t *up_raw, const uint8_t *down_t_raw, int ggml_type,
                           int h, int ff, const float *x, const int32_t *active,
                           int n_active, int act, float *out);

/* The same with the rows read from a file as the reference does
 * (ffn_flash.go:262-270: two ReadRowsParallel calls), tensors at the given
 * byte offsets. */
int refcpu_ffn_sparse_load_file(const char *path, int64_t up_offset, int64_t down_t_offset,
                                int ggml_type, int h, int ff, const float *x,
                                const int32_t *active, int n_active, int act, int nthreads,
                                float *out);

/* inference/forward.go:318-353 + 428-445 (dense ReLU/GELU path, no gate).
 * up_raw: [F rows x h]; down_raw: standard GGUF layout [h rows x F]. */
int refcpu_ffn_dense(const uint8_t *up_raw, const uint8_t *down_raw, int ggml_type, int h,
                     int ff, const float *x, int act, float *out);
/* ffnSwiGLU (forward.go:368-389): out = down @ (silu(gate @ x) * (up @ x)). */
int refcpu_ffn_swiglu(const uint8_t *gate_raw, const uint8_t *up_raw, const uint8_t *down_raw,
                      int ggml_type, int h, int ff, const float *x, float *out);

/* inference/window.go:21-245 -- NeuronCache. */
typedef struct refcpu_neuron_cache refcpu_neuron_cache;
refcpu_neuron_cache *refcpu_nc_new(int max_neurons, int hidden, int window, int ff,
                                   const uint8_t *up_raw, const uint8_t *down_t_raw,
                                   int ggml_type);
/* A cache whose loadRows reads the file at path (window.go:208-216, two
 * ReadRowsParallel calls with 32 threads). */
refcpu_neuron_cache *refcpu_nc_new_file(int max_neurons, int hidden, int window, int ff,
                                        const char *path, int64_t up_offset,
                                        int64_t down_t_offset, int ggml_type, int nthreads);
void refcpu_nc_free(refcpu_neuron_cache *c);
/* window.go:71-117.  n_loaded_out (optional) receives |toLoad|; load_list_out
 * (optional, capacity n_active) receives toLoad in the reference's order. */
int refcpu_nc_update(refcpu_neuron_cache *c, const int32_t *active, int n_active,
                     int *n_loaded_out, int32_t *load_list_out);
/* window.go:143-180 */
int refcpu_nc_ffn_forward(refcpu_neuron_cache *c, const float *x, const int32_t *active,
                          int n_active, int act, float *out);
int refcpu_nc_num_cached(const refcpu_neuron_cache *c);
/* window.go:121-128: 1 if neuron n is resident. */
int refcpu_nc_is_cached(const refcpu_neuron_cache *c, int n);

/* inference/moe_forward.go:32-150.  router [n_exp x hidden] f32.
 * gate/up: GGUF dims [hidden, eff, n_exp] (n_exp*eff rows of ByteSize(hidden));
 * down: dims [eff, hidden, n_exp] (n_exp*hidden rows of ByteSize(eff)).
 * ids_out/w_out (optional, [k]) receive the chosen experts and p/wsum in
 * accumulation order.  Returns 0, -1 on invalid hparams. */
int refcpu_moe_ffn(const float *router, const uint8_t *gate_raw, const uint8_t *up_raw,
                   const uint8_t *down_raw, int ggml_type, int hidden, int eff, int n_exp,
                   int k, const float *x, float *out, int32_t *ids_out, float *w_out);

/* Router stage of moe_forward.go:42-68 alone (softmax, descending sort with
 * ties to the lower index, top-k, renorm) on given logits. */
int refcpu_moe_route(const float *logits, int n_exp, int k, int32_t *ids_out, float *w_out);

/* Falcon-architecture decode on the sparse FFN path:
 * inference/ffn_flash.go:115-185 (ForwardFlash, forwardLayerFlash with the
 * parallel attention/FFN layout, ffnFlash path 2), inference/forward.go:206-310
 * (attention without biases or QK norm), :449-497 (embedding, RoPE),
 * kvcache/kvcache.go:25-82, tensor/ops.go:138-165 (LayerNorm).
 * Matrices are GGUF rows of type t; per-layer arrays are concatenated layer
 * after layer.  As the reference does at load, the embedding, attention and
 * LM-head matrices are dequantized to fp32 once in refcpu_falcon_new; the FFN
 * rows are dequantized per token (ffnSparseLoad).  refcpu_set_threads splits
 * the matvecs, the attention heads and the FFN rows over threads without
 * changing any result. */
typedef struct {
    int n_layers, hidden, n_heads, n_kv, head_dim, ff, vocab, max_seq, rank, act, t;
    float rope_base, eps;
    const uint8_t *embed;          /* vocab rows of ByteSize(hidden) */
    const float *norm_w, *norm_b;  /* [n_layers][hidden] */
    const uint8_t *wq, *wk, *wv;   /* [n_layers][n_heads*hd | n_kv*hd rows of ByteSize(hidden)] */
    const uint8_t *wo;             /* [n_layers][hidden rows of ByteSize(n_heads*hd)] */
    const float *pwup, *pwout;     /* [n_layers][rank x hidden], [n_layers][ff x rank] */
    const float *thr;              /* [n_layers] */
    const uint8_t *up, *down_t;    /* [n_layers][ff rows of ByteSize(hidden)] */
    const float *out_w, *out_b;    /* [hidden] */
    const uint8_t *lm_head;        /* vocab rows of ByteSize(hidden) */
} refcpu_falcon_params;
typedef struct refcpu_falcon refcpu_falcon;
refcpu_falcon *refcpu_falcon_new(const refcpu_falcon_params *p);
void refcpu_falcon_free(refcpu_falcon *m);
/* ForwardFlash(token, pos): logits [vocab]; n_active_out (optional) [n_layers].
 * The K/V of this token go to cache row SeqLen; returns 0, or -1 if the token
 * or SeqLen is out of range. */
int refcpu_falcon_forward(refcpu_falcon *m, int32_t token, int pos, float *logits,
                          int32_t *n_active_out);
/* The same, also writing every layer's predictor logits (predictor.go:57-73)
 * to pred_logits_out [n_layers x ff] when it is not NULL. */
int refcpu_falcon_forward_ex(refcpu_falcon *m, int32_t token, int pos, float *logits,
                             int32_t *n_active_out, float *pred_logits_out);
/* kvcache.go:55-57 (generate.go:94,119 call it after every token). */
void refcpu_falcon_commit(refcpu_falcon *m);
/* From the next forward on, the FFN rows of layer l are read from the GGUF
 * file at `path` (tensors at byte offsets up_off[l] and down_off[l], ff rows
 * of ByteSize(hidden) each) by a ReadRowsParallel pool of nthreads
 * (flash/storage.go:246-319, as ffn_flash.go:262-270 does) instead of from
 * p.up / p.down_t; the results are the same.  path NULL goes back to the
 * rows in memory.  Returns 0, or -1 when out of memory.  A forward whose rows
 * cannot be read returns -2. */
int refcpu_falcon_ffn_file(refcpu_falcon *m, const char *path, const int64_t *up_off,
                           const int64_t *down_off, int nthreads);
/* cmd/generate.go:197-205 */
int refcpu_argmax(const float *v, int n);

#ifdef __cplusplus
}
#endif
#endif
