// llg_window.hip -- sliding-window resident neuron set (inference/window.go).
//
// Device state per window (one FFN layer):
//   res[ff]       the number of the update that loaded n while n is resident
//                 (its bundle in row n of the resident buffer), else 0
//                                                      (the inCache map, window.go:27)
//   cnt[ff]       entries of the last k sets that hold n
//   ring[k+1][ff] the last k sets (k+1 slots, so the set of this update and
//                 the expiring one never share a slot)   (lastKActive, window.go:30)
//   state         [2] resident neurons (NumCached)
//   cntr[2]       loads of an update, in cntr[epoch & 1]
//   uslot[ff]     the update + FFN step's activations (64-bit, epoch-tagged)
//   resident      ff bundles of bstride bytes            (matrix, window.go:23)
//
// Neuron n always takes row n, so an update needs no slot allocation.  The
// update of the counts and the residency is split over workgroups, each
// working from the state at the start of the update and a bitmap of the
// listed set (win_update_part, llg_window_upd.hpp); during update e a neuron
// is resident at the start of the update exactly when res[n] is neither 0 nor
// e, so the update marks its loads (res = e) while the bundle copies and the
// FFN of the same launch still read the state at its start.  A plain update
// runs the copies (k_win_copy) and then the update (k_win_update); the
// update + FFN step runs the update beside the FFN in one launch (k_win_step,
// llg_sparse.hip), whose up rows copy each loaded bundle as they read it.
//
// Physical row order differs from the reference's swap-with-last order
// (window.go:188-204); it is unobservable, because FFNForward walks the
// active list, not the cache order (window.go:148,166).  The buffer holds
// every neuron's row, so the grow branch (window.go:222-232) is never needed.
#include "llg_common.hpp"
#include "llg_internal.hpp"
#include "llg_window_upd.hpp"

#include <vector>

struct LlgWindow {
    LlgObject *bundle;  // source bundle (the layer in HBM)
    int k, ff, head;    // head: ring slot of the next set
    int epoch;          // number of the last update (tags); starts at 1
    int32_t *res, *cnt, *ring, *ring_len, *ring_set, *state, *cntr;
    uint64_t *uslot;
    uint8_t *resident;
    long long bstride;
};

void llg_window_destroy(LlgDevice *d, LlgObject *o) {
    LlgWindow *w = reinterpret_cast<LlgWindow *>(o->ext);
    if (!w) return;
    hipFree(w->res);
    hipFree(w->uslot);
    hipFree(w->resident);
    llg_unref(d, w->bundle);
    delete w;
    o->ext = nullptr;
}

// The copies of a plain update: one wavefront per listed entry (grid-stride)
// copies the bundle of a neuron that is not resident into its row
// (loadRows, window.go:207-245).  A device list is not checked on the host,
// so the count is clamped to [0, ff] and an index outside [0, ff) is skipped:
// every access stays in bounds.
__global__ __launch_bounds__(256) void k_win_copy(LlgWinUpd u, const int32_t *__restrict__ active,
                                                  const int32_t *__restrict__ n_active_p, int ff,
                                                  long long bstride) {
    const int n_act = min(max(*n_active_p, 0), ff);
    const int lane = threadIdx.x & 63;
    const int n16 = (int)(bstride >> 4);
    for (int j = blockIdx.x * 4 + (threadIdx.x >> 6); j < n_act; j += gridDim.x * 4) {
        const int n = active[j];
        if (n < 0 || n >= ff || __builtin_amdgcn_readfirstlane((int)win_resident(u.res, n, u.epoch)))
            continue;
        const uint4 *sp = reinterpret_cast<const uint4 *>(u.src + (long long)n * bstride);
        uint4 *dp = reinterpret_cast<uint4 *>(u.dst + (long long)n * bstride);
        for (int c = lane; c < n16; c += 64) dp[c] = sp[c];
    }
}

// The counts and the residency of a plain update, part blockIdx.x of
// gridDim.x (LDS: the bitmap of the listed set).
__global__ __launch_bounds__(256) void k_win_update(LlgWinUpd u, const int32_t *__restrict__ active,
                                                    const int32_t *__restrict__ n_active_p,
                                                    int ff) {
    extern __shared__ uint32_t bm[];
    win_update_part(u, active, min(max(*n_active_p, 0), ff), ff, blockIdx.x, gridDim.x, bm);
}

// Workgroups of an update (each takes every WIN_UPD_PARTS-th entry).
#define WIN_UPD_PARTS 16

static LlgWindow *get_window(LlgDevice *d, int64_t h) {
    LlgObject *o = llg_get(d, h, LLG_KIND_WINDOW);
    return o ? reinterpret_cast<LlgWindow *>(o->ext) : nullptr;
}

// Number of the update after `e`.  Loads are counted in cntr[epoch & 1] and
// each update clears the other counter for the next one, so consecutive
// numbers must alternate in parity, across the wrap too: after 0x7FFFFFFF
// (odd) comes 2, never 1 (0 marks a neuron that is not resident).
constexpr int llg_next_epoch(int e) { return e == 0x7FFFFFFF ? 2 : e + 1; }
static_assert(llg_next_epoch(0) == 1 && llg_next_epoch(1) == 2, "updates are numbered from 1");
static_assert(llg_next_epoch(0x7FFFFFFF) == 2 && llg_next_epoch(0x7FFFFFFE) == 0x7FFFFFFF,
              "the wrap keeps 0 reserved");
static_assert(((llg_next_epoch(0x7FFFFFFF) ^ 0x7FFFFFFF) & 1) &&
                  ((llg_next_epoch(0x7FFFFFFE) ^ 0x7FFFFFFE) & 1) &&
                  ((llg_next_epoch(llg_next_epoch(0x7FFFFFFF)) ^ llg_next_epoch(0x7FFFFFFF)) & 1),
              "consecutive updates alternate in parity across the wrap");

// The next update: numbers it, and names its ring slot and the expiring one.
// When the numbers wrap, the activation slots are cleared, so that no slot
// keeps a tag from 2^31 updates ago (a neuron that has stayed resident since
// then counts one load more).
static LlgWinUpd next_update(LlgWindow *w, hipStream_t st) {
    const bool wraps = w->epoch == 0x7FFFFFFF;
    w->epoch = llg_next_epoch(w->epoch);
    if (wraps) (void)hipMemsetAsync(w->uslot, 0, (size_t)w->ff * 8, st);
    const int e = (w->head + 1) % (w->k + 1);  // the set of k updates ago
    const size_t ff = (size_t)w->ff;
    LlgWinUpd u;
    u.src = w->bundle->d;
    u.dst = w->resident;
    u.res = w->res;
    u.cnt = w->cnt;
    u.state = w->state;
    u.cntr = w->cntr;
    u.ring_new = w->ring + (size_t)w->head * ff;
    u.ring_len_new = w->ring_len + w->head;
    u.ring_set_new = w->ring_set + w->head;
    u.ring_exp = w->ring + (size_t)e * ff;
    u.ring_len_exp = w->ring_len + e;
    u.ring_set_exp = w->ring_set + e;
    u.uslot = w->uslot;
    u.epoch = w->epoch;
    u.check = 0;
    w->head = (w->head + 1) % (w->k + 1);
    return u;
}

static int window_update_enqueue(LlgDevice *d, LlgWindow *w, const int32_t *d_active,
                                 const int32_t *d_n_active, int max_active) {
    hipStream_t st = llg_dev_stream(d);
    const LlgWinUpd u = next_update(w, st);
    const int grid = std::max(1, std::min((std::max(max_active, 1) + 3) / 4, 2048));
    hipLaunchKernelGGL(k_win_copy, dim3(grid), dim3(256), 0, st, u, d_active, d_n_active, w->ff,
                       w->bstride);
    hipLaunchKernelGGL(k_win_update, dim3(WIN_UPD_PARTS), dim3(256),
                       (size_t)win_bitmap_words(w->ff) * 4, st, u, d_active, d_n_active, w->ff);
    LLG_LAUNCH_CHECK(d, "window_update");
    return 0;
}

extern "C" {

int llg_hip_window_create(LlgHipDevice h, int64_t hb, int k, int64_t *win) {
    LlgDevice *d = llg_dev(h);
    if (!d) return LLG_E_NODEV;
    LlgObject *b = llg_get(d, hb, LLG_KIND_BUNDLE);
    if (!b) return llg_set_error(d, LLG_E_HANDLE, "window_create: unknown bundle");
    if (k < 1 || !win) return llg_set_error(d, LLG_E_ARG, "window_create: k must be >= 1");
    LlgWindow *w = new LlgWindow();
    w->bundle = b;
    w->k = k;
    w->ff = b->rows;
    w->head = 0;
    w->bstride = b->stride;
    const size_t ff = (size_t)w->ff, slots = (size_t)k + 1;
    // one allocation for the int32 state arrays
    const size_t n_ints = ff * 2 + slots * ff + 2 * slots + 4 + 2;
    int32_t *m = nullptr;
    if (hipMalloc(&m, n_ints * 4) != hipSuccess) {
        delete w;
        return llg_set_error(d, LLG_E_NOMEM, "window_create: state allocation failed");
    }
    w->res = m;  // 0: nothing resident
    w->cnt = m + ff;
    w->ring = w->cnt + ff;
    w->ring_len = w->ring + slots * ff;
    w->ring_set = w->ring_len + slots;
    w->state = w->ring_set + slots;
    w->cntr = w->state + 4;
    w->epoch = 0;
    w->uslot = nullptr;
    w->resident = nullptr;
    if (hipMalloc(&w->uslot, ff * 8) != hipSuccess ||
        hipMalloc(&w->resident, ff * w->bstride) != hipSuccess) {
        hipFree(m);
        if (w->uslot) hipFree(w->uslot);
        delete w;
        return llg_set_error(d, LLG_E_NOMEM, "window_create: resident buffer allocation failed");
    }
    hipStream_t st = llg_dev_stream(d);
    hipError_t e = hipMemsetAsync(m, 0, n_ints * 4, st);
    if (e == hipSuccess) e = hipMemsetAsync(w->uslot, 0, ff * 8, st);  // tag 0: no update
    if (e == hipSuccess) e = hipStreamSynchronize(st);
    if (e != hipSuccess) {
        hipFree(m);
        hipFree(w->uslot);
        hipFree(w->resident);
        delete w;
        return llg_hip_error(d, e, "window_create");
    }
    llg_ref(b);  // the window reads the bundle until it is destroyed
    LlgObject *o = new LlgObject();
    o->kind = LLG_KIND_WINDOW;
    o->d = nullptr;
    o->bytes = (size_t)w->ff * w->bstride;
    o->fmt = b->fmt;
    o->rows = w->ff;
    o->stride = w->bstride;
    o->ext = w;
    *win = llg_register(d, o);
    return 0;
}

int llg_hip_window_update(LlgHipDevice h, int64_t hw, const int32_t *active, int n_active,
                          int *n_loaded, int *n_resident) {
    LlgDevice *d = llg_dev(h);
    if (!d) return LLG_E_NODEV;
    LlgWindow *w = get_window(d, hw);
    if (!w) return llg_set_error(d, LLG_E_HANDLE, "window_update: unknown window");
    if (n_active < 0 || (n_active > 0 && !active))
        return llg_set_error(d, LLG_E_ARG, "window_update: bad active list");
    if (n_active > w->ff) return llg_set_error(d, LLG_E_ARG, "window_update: too many neurons");
    std::vector<uint8_t> seen((size_t)w->ff, 0);
    for (int j = 0; j < n_active; j++) {
        if (active[j] < 0 || active[j] >= w->ff)
            return llg_set_error(d, LLG_E_RANGE, "row %d out of range [0,%d)", active[j], w->ff);
        if (seen[active[j]]) return llg_set_error(d, LLG_E_ARG, "window_update: duplicate neuron");
        seen[active[j]] = 1;
    }
    int rc;
    const long long o_n = llg_align((long long)n_active * 4 + 4, 256);
    uint8_t *ws = (uint8_t *)llg_ws(d, o_n + 256, &rc);
    if (rc) return rc;
    const int32_t n32 = n_active;
    if ((rc = llg_h2d(d, ws, active, (size_t)n_active * 4))) return rc;
    if ((rc = llg_h2d(d, ws + o_n, &n32, 4))) return rc;
    if ((rc = window_update_enqueue(d, w, (const int32_t *)ws, (const int32_t *)(ws + o_n),
                                    n_active)))
        return rc;
    int32_t st[6];  // state[0..3] and cntr[0..1]
    if ((rc = llg_d2h(d, st, w->state, sizeof st))) return rc;
    if ((rc = llg_sync_dev(d))) return rc;
    if (n_loaded) *n_loaded = st[4 + (w->epoch & 1)];
    if (n_resident) *n_resident = st[2];
    return 0;
}

int llg_hip_window_ffn(LlgHipDevice h, int64_t hw, const float *x, const int32_t *active,
                       int n_active, int act, float *out) {
    LlgDevice *d = llg_dev(h);
    if (!d) return LLG_E_NODEV;
    LlgWindow *w = get_window(d, hw);
    if (!w) return llg_set_error(d, LLG_E_HANDLE, "window_ffn: unknown window");
    const int hd = w->bundle->fmt.cols;
    if (!x || !out || n_active < 0 || (n_active > 0 && !active))
        return llg_set_error(d, LLG_E_ARG, "window_ffn: bad arguments");
    if (int rc = llg_check_act(d, act)) return rc;
    for (int j = 0; j < n_active; j++)
        if (active[j] < 0 || active[j] >= w->ff)
            return llg_set_error(d, LLG_E_RANGE, "row %d out of range [0,%d)", active[j], w->ff);
    if (n_active == 0) {
        for (int i = 0; i < hd; i++) out[i] = 0.0f;
        return 0;
    }
    const long long o_act = llg_align((long long)hd * 4, 256);
    const long long o_n = o_act + llg_align((long long)n_active * 4, 256);
    const long long o_out = o_n + 256;
    const long long o_ws = o_out + llg_align((long long)hd * 4, 256);
    int rc;
    uint8_t *ws = (uint8_t *)llg_ws(d, o_ws + llg_sparse_ws_bytes(n_active), &rc);
    if (rc) return rc;
    const int32_t n32 = n_active;
    if ((rc = llg_h2d(d, ws, x, (size_t)hd * 4))) return rc;
    if ((rc = llg_h2d(d, ws + o_act, active, (size_t)n_active * 4))) return rc;
    if ((rc = llg_h2d(d, ws + o_n, &n32, 4))) return rc;
    rc = llg_sparse_enqueue(d, w->resident, w->bstride, w->bundle->fmt, w->res,
                            (const float *)ws, (const int32_t *)(ws + o_act),
                            (const int32_t *)(ws + o_n), n_active, w->ff, act,
                            (float *)(ws + o_out), ws + o_ws);
    if (rc) return rc;
    if ((rc = llg_d2h(d, out, ws + o_out, (size_t)hd * 4))) return rc;
    return llg_sync_dev(d);
}

int llg_hipd_window_step(LlgHipDevice h, int64_t hw, const float *d_x, const int32_t *d_active,
                         const int32_t *d_n_active, int act, float *d_out) {
    LlgDevice *d = llg_dev(h);
    if (!d) return LLG_E_NODEV;
    LlgWindow *w = get_window(d, hw);
    if (!w) return llg_set_error(d, LLG_E_HANDLE, "window_step: unknown window");
    if (!d_x || !d_active || !d_n_active || !d_out)
        return llg_set_error(d, LLG_E_ARG, "window_step: null pointer");
    if (int rc = llg_check_act(d, act)) return rc;
    LlgWinUpd u = next_update(w, llg_dev_stream(d));
    u.check = llg_dev_check(d);
    return llg_win_step_enqueue(d, u, w->bundle->fmt, w->bstride, d_x, d_active, d_n_active,
                                w->ff, w->ff, act, d_out);
}

int llg_hip_window_resident(LlgHipDevice h, int64_t hw, uint8_t *resident, int *n_resident) {
    LlgDevice *d = llg_dev(h);
    if (!d) return LLG_E_NODEV;
    LlgWindow *w = get_window(d, hw);
    if (!w) return llg_set_error(d, LLG_E_HANDLE, "window_resident: unknown window");
    std::vector<int32_t> res((size_t)w->ff);
    int32_t st[4];
    int rc;
    if ((rc = llg_d2h(d, res.data(), w->res, (size_t)w->ff * 4))) return rc;
    if ((rc = llg_d2h(d, st, w->state, sizeof st))) return rc;
    if ((rc = llg_sync_dev(d))) return rc;
    if (resident)
        for (int i = 0; i < w->ff; i++) resident[i] = res[i] != 0 ? 1 : 0;
    if (n_resident) *n_resident = st[2];
    return 0;
}

}  // extern "C"
