// llg_window.hip -- sliding-window resident neuron set (inference/window.go).
//
// Device state per window (one FFN layer):
//   slot_of[ff]   n when neuron n is resident (its bundle in row n of the
//                 resident buffer), else -1            (the inCache map, window.go:27)
//   cnt[ff]       entries of the last k sets that hold n
//   cur_ep[ff]    the number of the last update whose set held n
//   fresh[ff]     the number of the update that last loaded n
//   ring[k+1][ff] the last k sets (k+1 slots, so the set of this update and
//                 the expiring one never share a slot)   (lastKActive, window.go:30)
//   state         [2] resident neurons (NumCached), [3] loads of the last update
//   resident      ff bundles of bstride bytes            (matrix, window.go:23)
//
// Neuron n always takes row n, so an update needs no slot allocation and
// splits into per-entry steps (llg_window_upd.hpp) over two launches:
//   1. each entry of the set is recorded, marked and counted; each entry of
//      the expiring set is uncounted (window.go:73-80); a listed neuron that
//      is not resident is copied from the layer's bundle into its row
//      (loadRows, window.go:207-245);
//   2. an expiring neuron whose count is 0 and that the set does not hold is
//      evicted (window.go:84-95); the loaded ones become resident.
// A plain update runs them as k_win_update1 / k_win_update2; the update + FFN
// step folds them into the list FFN's two launches (llg_sparse.hip), whose
// first launch reads every loaded neuron's up row as it copies the bundle.
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
    int32_t *slot_of, *cnt, *cur_ep, *fresh, *ring, *ring_len, *ring_set, *state, *cntr;
    uint8_t *resident;
    long long bstride;
};

void llg_window_destroy(LlgDevice *d, LlgObject *o) {
    LlgWindow *w = reinterpret_cast<LlgWindow *>(o->ext);
    if (!w) return;
    hipFree(w->slot_of);
    hipFree(w->resident);
    llg_unref(d, w->bundle);
    delete w;
    o->ext = nullptr;
}

// Step 1 of a plain update: one wavefront per listed entry (grid-stride);
// every thread also takes a share of the expiring set.  A device list is not
// checked on the host, so the count is clamped to [0, ff] and an index outside
// [0, ff) is recorded as -1 and skipped: every access stays in bounds.
__global__ __launch_bounds__(256) void k_win_update1(LlgWinUpd u, const int32_t *__restrict__ active,
                                                     const int32_t *__restrict__ n_active_p,
                                                     int ff, long long bstride) {
    const int n_act = min(max(*n_active_p, 0), ff);
    win_expire_all(u, n_act, ff, blockIdx.x * blockDim.x + threadIdx.x, gridDim.x * blockDim.x);
    const int lane = threadIdx.x & 63;
    const int n16 = (int)(bstride >> 4);
    for (int j = blockIdx.x * 4 + (threadIdx.x >> 6); j < n_act; j += gridDim.x * 4) {
        int n = active[j];
        n = n >= 0 && n < ff ? n : -1;
        int ld = 0;
        if (lane == 0) ld = win_note_active(u, j, n);
        if (__builtin_amdgcn_readfirstlane(ld)) {
            const uint4 *sp = reinterpret_cast<const uint4 *>(u.src + (long long)n * bstride);
            uint4 *dp = reinterpret_cast<uint4 *>(u.dst + (long long)n * bstride);
            for (int c = lane; c < n16; c += 64) dp[c] = sp[c];
            if (lane == 0) win_note_load(u, n);
        }
    }
}

// Step 2 of a plain update.
__global__ __launch_bounds__(256) void k_win_update2(LlgWinUpd u,
                                                     const int32_t *__restrict__ n_active_p,
                                                     int ff) {
    win_finish_all(u, min(max(*n_active_p, 0), ff), ff, blockIdx.x * blockDim.x + threadIdx.x,
                   gridDim.x * blockDim.x);
}

static LlgWindow *get_window(LlgDevice *d, int64_t h) {
    LlgObject *o = llg_get(d, h, LLG_KIND_WINDOW);
    return o ? reinterpret_cast<LlgWindow *>(o->ext) : nullptr;
}

// Number of the update after `e`.  Loads are counted in cntr[epoch & 1] and
// each update clears the other counter for the next one, so consecutive
// numbers must alternate in parity, across the wrap too: after 0x7FFFFFFF
// (odd) comes 2, never 1 (0 stays "never listed").
constexpr int llg_next_epoch(int e) { return e == 0x7FFFFFFF ? 2 : e + 1; }
static_assert(llg_next_epoch(0) == 1 && llg_next_epoch(1) == 2, "updates are numbered from 1");
static_assert(llg_next_epoch(0x7FFFFFFF) == 2 && llg_next_epoch(0x7FFFFFFE) == 0x7FFFFFFF,
              "the wrap keeps 0 reserved");
static_assert(((llg_next_epoch(0x7FFFFFFF) ^ 0x7FFFFFFF) & 1) &&
                  ((llg_next_epoch(0x7FFFFFFE) ^ 0x7FFFFFFE) & 1) &&
                  ((llg_next_epoch(llg_next_epoch(0x7FFFFFFF)) ^ llg_next_epoch(0x7FFFFFFF)) & 1),
              "consecutive updates alternate in parity across the wrap");

// The folded update of the next set: numbers it, and names its ring slot and
// the expiring one.
static LlgWinUpd next_update(LlgWindow *w) {
    w->epoch = llg_next_epoch(w->epoch);
    const int e = (w->head + 1) % (w->k + 1);  // the set of k updates ago
    const size_t ff = (size_t)w->ff;
    LlgWinUpd u;
    u.src = w->bundle->d;
    u.dst = w->resident;
    u.slot_of = w->slot_of;
    u.cnt = w->cnt;
    u.cur_ep = w->cur_ep;
    u.fresh = w->fresh;
    u.state = w->state;
    u.cntr = w->cntr;
    u.ring_new = w->ring + (size_t)w->head * ff;
    u.ring_len_new = w->ring_len + w->head;
    u.ring_set_new = w->ring_set + w->head;
    u.ring_exp = w->ring + (size_t)e * ff;
    u.ring_len_exp = w->ring_len + e;
    u.ring_set_exp = w->ring_set + e;
    u.epoch = w->epoch;
    w->head = (w->head + 1) % (w->k + 1);
    return u;
}

static int window_update_enqueue(LlgDevice *d, LlgWindow *w, const int32_t *d_active,
                                 const int32_t *d_n_active, int max_active) {
    hipStream_t st = llg_dev_stream(d);
    const LlgWinUpd u = next_update(w);
    const int grid = std::max(1, std::min((std::max(max_active, 1) + 3) / 4, 2048));
    hipLaunchKernelGGL(k_win_update1, dim3(grid), dim3(256), 0, st, u, d_active, d_n_active, w->ff,
                       w->bstride);
    hipLaunchKernelGGL(k_win_update2, dim3(grid), dim3(256), 0, st, u, d_n_active, w->ff);
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
    const size_t n_ints = ff * 4 + slots * ff + 2 * slots + 4 + 2;
    int32_t *m = nullptr;
    if (hipMalloc(&m, n_ints * 4) != hipSuccess) {
        delete w;
        return llg_set_error(d, LLG_E_NOMEM, "window_create: state allocation failed");
    }
    w->slot_of = m;
    w->cnt = m + ff;
    w->cur_ep = w->cnt + ff;  // 0: never listed (updates are numbered from 1)
    w->fresh = w->cur_ep + ff;
    w->ring = w->fresh + ff;
    w->ring_len = w->ring + slots * ff;
    w->ring_set = w->ring_len + slots;
    w->state = w->ring_set + slots;
    w->cntr = w->state + 4;
    w->epoch = 0;
    if (hipMalloc(&w->resident, ff * w->bstride) != hipSuccess) {
        hipFree(m);
        delete w;
        return llg_set_error(d, LLG_E_NOMEM, "window_create: resident buffer allocation failed");
    }
    hipStream_t st = llg_dev_stream(d);
    hipError_t e = hipMemsetAsync(m, 0, n_ints * 4, st);
    if (e == hipSuccess) e = hipMemsetAsync(w->slot_of, 0xFF, ff * 4, st);  // -1: nothing resident
    if (e == hipSuccess) e = hipStreamSynchronize(st);
    if (e != hipSuccess) {
        hipFree(m);
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
    int32_t st[4];
    if ((rc = llg_d2h(d, st, w->state, sizeof st))) return rc;
    if ((rc = llg_sync_dev(d))) return rc;
    if (n_loaded) *n_loaded = st[3];
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
    rc = llg_sparse_enqueue(d, w->resident, w->bstride, w->bundle->fmt, w->slot_of,
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
    int rc;
    uint8_t *ws = (uint8_t *)llg_ws(d, llg_sparse_ws_bytes(w->ff), &rc);
    if (rc) return rc;
    const LlgWinUpd u = next_update(w);
    return llg_sparse_enqueue(d, w->resident, w->bstride, w->bundle->fmt, w->slot_of, d_x,
                              d_active, d_n_active, w->ff, w->ff, act, d_out, ws, &u);
}

int llg_hip_window_resident(LlgHipDevice h, int64_t hw, uint8_t *resident, int *n_resident) {
    LlgDevice *d = llg_dev(h);
    if (!d) return LLG_E_NODEV;
    LlgWindow *w = get_window(d, hw);
    if (!w) return llg_set_error(d, LLG_E_HANDLE, "window_resident: unknown window");
    std::vector<int32_t> slots((size_t)w->ff);
    int32_t st[4];
    int rc;
    if ((rc = llg_d2h(d, slots.data(), w->slot_of, (size_t)w->ff * 4))) return rc;
    if ((rc = llg_d2h(d, st, w->state, sizeof st))) return rc;
    if ((rc = llg_sync_dev(d))) return rc;
    if (resident)
        for (int i = 0; i < w->ff; i++) resident[i] = slots[i] >= 0 ? 1 : 0;
    if (n_resident) *n_resident = st[2];
    return 0;
}

}  // extern "C"
