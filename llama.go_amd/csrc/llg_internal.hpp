// llg_internal.hpp -- enqueue functions shared between translation units.
#pragma once
#include "llg_common.hpp"

// Predictor (llg_predictor.hip)
int llg_predict_ws_bytes(int rank, int ff);
int llg_predict_enqueue(LlgDevice *d, LlgObject *wup, LlgObject *wout, LlgObject *bias,
                        const float *d_a, float thr, int32_t *d_active, int32_t *d_n_active,
                        float *d_logits, uint8_t *ws);
int llg_check_predictor(LlgDevice *d, int64_t hwup, int64_t hwout, int64_t hbias,
                        LlgObject **wup, LlgObject **wout, LlgObject **bias);

// Sparse FFN over bundles (llg_ffn.hip).  Neuron n's bundle is at
// base + (slot_of ? slot_of[n] : n) * bstride.  max_active bounds *d_n_active.
size_t llg_sparse_ws_bytes(int max_active);
int llg_sparse_enqueue(LlgDevice *d, const uint8_t *base, long long bstride, const RowFmt &f,
                       const int32_t *slot_of, const float *d_x, const int32_t *d_active,
                       const int32_t *d_n_active, int max_active, int act, float *d_out,
                       uint8_t *ws);

// Dense quantized matvec y[rows] = act(W . x) (llg_ffn.hip); act < 0 = none.
int llg_matvec_enqueue(LlgDevice *d, const LlgObject *w, const float *d_x, int act, float *d_y);
