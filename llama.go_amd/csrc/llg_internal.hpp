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
// K1 of the predictor: hidden partials into ws; also zeroes the given targets.
// zero_out[0..zero_n) is cleared, or, with add_to, accumulated (+= add_to[i]).
int llg_pred_hidden_enqueue(LlgDevice *d, LlgObject *wup, const float *d_a, uint8_t *ws,
                            float **partial, unsigned long long **mask, int *psplit,
                            float *zero_out, int zero_n, int32_t *zero_ctr, int n_ctr,
                            int32_t *zero_extra, const float *add_to = nullptr);
// Hidden partials + tile masks (k_pred_hidden, k_pred_logits); also clears
// zero_out[0..zero_n) and *zero_extra for the kernels that follow.
int llg_pred_masks_enqueue(LlgDevice *d, LlgObject *wup, LlgObject *wout, LlgObject *bias,
                           const float *d_a, float thr, uint8_t *ws,
                           unsigned long long **mask_out, float *zero_out, int zero_n,
                           int32_t *zero_extra);
// Where the hidden partials ([split][rank] floats) and the tile masks sit in
// a predictor workspace; the number of partials per hidden unit.
void llg_pred_ws_layout(uint8_t *ws, int rank, float **partial, unsigned long long **mask);
int llg_pred_split();
// Logits, masks and the active list from hidden partials already in ws.
int llg_pred_logits_enqueue(LlgDevice *d, LlgObject *wout, LlgObject *bias, float thr,
                            uint8_t *ws, int32_t *d_active, int32_t *d_n_active,
                            float *d_logits);
// Ascending active list from 64-bit tile masks (one workgroup).
int llg_compact_enqueue(LlgDevice *d, const unsigned long long *mask, int n_tiles,
                        int32_t *d_active, int32_t *d_n_active);

// Sparse FFN over bundles (llg_sparse.hip).  Neuron n's bundle is at
// base + n * bstride.  max_active bounds *d_n_active.
size_t llg_sparse_ws_bytes(int max_active);
// The activations of model.ActivationType (model.go:97-103) an entry point
// accepts; anything else is an argument error.
inline bool llg_act_ok(int act) {
    return act == LLG_ACT_RELU || act == LLG_ACT_GELU || act == LLG_ACT_SILU;
}
inline int llg_check_act(LlgDevice *d, int act) {
    return llg_act_ok(act) ? 0 : llg_set_error(d, LLG_E_ARG, "activation %d is not ReLU, GELU or SiLU", act);
}

// One update (number `epoch`) of a window (llg_window.hip, window.go:71-117).
// Neuron n lives in row n of the resident buffer dst.  res[n] is the number of
// the update that loaded n, 0 when n is not resident; during update e, n is
// resident at the start of the update exactly when res[n] is neither 0 nor e
// (llg_window_upd.hpp), so the update can mark its loads while readers of the
// same launch still see the state at its start.  cnt[n]: entries of the last
// k sets that hold n; state[2]: resident neurons.  ring_new receives this
// update's set, ring_exp holds the expiring one (set k updates ago; its
// *ring_set_exp is 0 until the ring has wrapped).  uslot: the update + FFN
// step's activations, one 64-bit slot per list entry, tagged with the update's
// number (llg_pred_tile.hpp).  cntr[2]: the loads of an update are counted in
// cntr[epoch & 1] (consecutive update numbers alternate in parity).
struct LlgWinUpd {
    const uint8_t *src;
    uint8_t *dst;
    int32_t *res, *cnt, *state, *cntr;
    int32_t *ring_new, *ring_len_new, *ring_set_new;
    const int32_t *ring_exp, *ring_len_exp, *ring_set_exp;
    uint64_t *uslot;
    int epoch;
    int check;  // llg_dev_check: every entry's activation computed by the down role after its wait
};
// max_active: capacity of the list and of the pair workspace (the count read
// on the device is clamped to it); n_rows: the neurons of the bundle or window
// (an index outside [0, n_rows) counts as absent).  res (optional): a window's
// residency (a neuron with res[n] == 0 is not resident and keeps activation 0,
// window.go:150-152); the rows are then base + n * bstride, as without res.
int llg_sparse_enqueue(LlgDevice *d, const uint8_t *base, long long bstride, const RowFmt &f,
                       const int32_t *res, const float *d_x, const int32_t *d_active,
                       const int32_t *d_n_active, int max_active, int n_rows, int act,
                       float *d_out, uint8_t *ws);
// The window's update + FFN step in one launch (k_win_step): the FFN over the
// listed neurons (loaded ones read from u.src and copied to their rows) and
// update u.epoch of the counts and the residency.  cap: the list capacity
// (the device count is clamped to it); n_rows: the window's neurons.
int llg_win_step_enqueue(LlgDevice *d, const LlgWinUpd &u, const RowFmt &f, long long bstride,
                         const float *d_x, const int32_t *d_active, const int32_t *d_n_active,
                         int cap, int n_rows, int act, float *d_out);

// Dense quantized matvec y[rows] = act(W . x) (llg_ffn.hip); act < 0 = none.
// part: room for llg_matvec_part_bytes(w, act) (column-chunked rows keep
// their partial sums there, added in chunk order); may be null when that is 0.
int llg_matvec_enqueue(LlgDevice *d, const LlgObject *w, const float *d_x, int act, float *d_y,
                       float *part);
size_t llg_matvec_part_bytes(const LlgObject *w, int act);
// The attention-output matvec y = W . x, x the merge of the split attention
// output (LlgAttnParts).  With pf (LlgPredFold; W's rows must fit one
// workgroup's staged x, llg_matvec_fold_ok): y may be null, pf.resid += W . x,
// and the fold tasks' partial sums.  part: as for llg_matvec_enqueue.
bool llg_matvec_fold_ok(const LlgObject *w);
int llg_matvec_attn_enqueue(LlgDevice *d, const LlgObject *w, const LlgAttnParts &ap, float *d_y,
                            float *part, const LlgPredFold *pf);
// y = W . LayerNorm((x_in + a1) + a2), the residual sum and the normed row
// also written to ln.x_out / ln.normed_out (llg_stage_ln).
int llg_matvec_ln_enqueue(LlgDevice *d, const LlgObject *w, const LlgLnArgs &ln, float *d_y);

// Predictor-fused sparse FFN (ffnFlash path 2) (llg_sparse.hip).
// nb: 32-element blocks of the bundle rows (the tiles' partial outputs).
size_t llg_fused_ws_bytes(int rank, int ff, int nb);
// sync: a sync area of LLG_SYNC_BYTES (the predictor then runs inside the tile
// launch), or null (a separate predictor kernel first).
int llg_fused_enqueue(LlgDevice *d, LlgObject *wup, LlgObject *wout, LlgObject *bias,
                      LlgObject *b, const float *d_a, const float *d_x, float thr, int act,
                      float *d_out, int32_t *d_active, int32_t *d_n_active, uint8_t *ws,
                      uint8_t *sync, const float *d_out_add = nullptr,
                      float2 *d_stats = nullptr);
// The same after the hidden partials are in ws (llg_pred_ws_layout): the
// tile kernel and the partial-sum kernel; accumulate: d_out += the FFN output.
// d_stats (optional): per 32 outputs, (sum, M2) of d_out as written (LlgLnArgs).
int llg_fused_tail_enqueue(LlgDevice *d, LlgObject *wout, LlgObject *bias, LlgObject *b,
                           const float *d_x, float thr, int act, float *d_out,
                           int32_t *d_active, int32_t *d_n_active, uint8_t *ws, bool accumulate,
                           float2 *d_stats = nullptr);

// The sparse step of a Falcon layer with Wo and the predictor in the tile
// launch.  The attention kernel left pd[s][h][j] = P[j][head h] . acc_s per
// split s and head h (P = WUp . Wo, rank rows of Wo's width) beside the
// splits' (m, l) in ap.  The launch's first workgroups merge them into the
// predictor's hidden units (as the attention splits merge) and hand them to
// the tile workgroups through the sync area (sync, LLG_SYNC_BYTES); its last
// workgroups stage the attention output and add Wo . attn into d_resid (x +=
// attnOut, ffn_flash.go:161); then k_tile_reduce adds the FFN output into
// d_resid (x += ffnOut) with its block statistics.  llg_fused_wo_ok: whether
// Wo's type and sizes allow it.
bool llg_fused_wo_ok(const LlgObject *wo, int rank, int hidden);
int llg_fused_wo_enqueue(LlgDevice *d, const LlgObject *wo, const LlgAttnParts &ap,
                         const float *pd, LlgObject *wout, LlgObject *bias, LlgObject *b,
                         const float *d_x, float thr, int act, float *d_resid,
                         int32_t *d_n_active, uint8_t *ws, uint8_t *sync, float2 *d_stats);

// MoE prefill as grouped MFMA GEMMs (llg_moe_gemm.hip).
bool llg_moe_gemm_supported(int type, int hidden, int eff, int n_tok);
size_t llg_moe_gemm_ws_bytes(int n_tok, int k, int n_exp, int hidden, int eff);
int llg_moe_gemm_enqueue(LlgDevice *d, const LlgObject *gate, const LlgObject *up,
                         const LlgObject *down, int n_exp, int k, int hidden, int eff,
                         const float *d_x, int n_tok, const int32_t *ids, const float *w,
                         float *d_out, uint8_t *ws);
