// llg_window.hip -- sliding-window resident neuron set (inference/window.go).
//
// Device state per window (one FFN layer):
//   slot_of[ff]   resident slot of neuron n, or -1      (the inCache map, window.go:27)
//   cnt[ff]       how many of the k ring slots hold n
//   ring[k][ff]   the last k active sets, len/set flags   (lastKActive, window.go:30)
//   free stack    slots released by evictions; hw = slots ever handed out
//   fresh[ff]     the number of the update that last loaded n
//   resident      cap bundles of bstride bytes            (matrix, window.go:23)
//
// Update (window.go:71-117), one workgroup:
//   A. if the expiring slot is set: cnt[n]-- for its neurons
//   B. the active neurons are marked in an LDS bitmap (cur)
//   C. neurons of the expiring slot with cnt == 0 and !cur are evicted
//      (window.go:89-94): their slot goes on the free stack
//   D. active neurons without a slot form toLoad, in active order
//      (window.go:98-103); a block scan gives each its index k, and it takes
//      free slot top-1-k, or hw + (k - n_free) once the stack is empty
//   E. cnt[n]++, the set is recorded and the head advances
//      (window.go:113-114)
// then the toLoad bundles are copied from the layer's bundle into their
// resident slots (loadRows, window.go:207-245): by k_window_gather after a
// plain update, or, in the update + FFN step, by k_list_up as it reads each
// loaded neuron's up row (fresh[n] == this update's number), so the step
// takes no separate copy launch and reads no copied row back.
//
// Physical slot order differs from the reference's swap-with-last order
// (window.go:188-204); it is unobservable, because FFNForward walks the
// active list, not the cache order (window.go:148,166).  Capacity is ff slots,
// which bounds the union of any k active sets, so the grow branch
// (window.go:222-232) is never needed.
#include "llg_common.hpp"
#include "llg_internal.hpp"

#include <vector>

struct LlgWindow {
    LlgObject *bundle;  // source bundle (the layer in HBM)
    int k, ff, head;
    int cap;
    int epoch;  // number of the last update (fresh tags); starts at 1
    int32_t *slot_of, *cnt, *ring, *ring_len, *ring_set;
    int32_t *free_stack, *fresh;
    int32_t *state;      // [0]=free_top [1]=hw [2]=n_res [3]=n_loaded
    int32_t *load_list;  // [ff] pairs (neuron, slot)
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

#define WIN_EVCAP 2048  // evicted slots of one update also kept in LDS

// Round trips are the cost of this one-workgroup kernel, so the first 1024
// entries of both lists are loaded up front (with their slots and the
// decrement of cnt) and kept in registers; the current set is an
// LDS bitmap (ff bits); this update's evictions go on the global free stack
// and, up to WIN_EVCAP, into LDS, where the slot assignment reads them.
// A device list is not checked on the host, so every access stays in bounds
// whatever it holds: the count is clamped to [0, ff], an index outside
// [0, ff) is recorded as -1 and skipped, the free stack never grows past ff
// entries and no slot at or past ff is handed out (such a neuron stays
// non-resident).  The results of such a list are meaningless, but safe.
__global__ __launch_bounds__(1024) void k_window_update(
    int32_t *__restrict__ slot_of, int32_t *__restrict__ cnt, int32_t *__restrict__ ring,
    int32_t *__restrict__ ring_len, int32_t *__restrict__ ring_set,
    int32_t *__restrict__ free_stack, int32_t *__restrict__ state,
    int32_t *__restrict__ load_list, int32_t *__restrict__ fresh, int epoch,
    const int32_t *__restrict__ active, const int32_t *__restrict__ n_active_p, int head,
    int ff) {
    extern __shared__ uint32_t curbits[];  // [ceil(ff / 32)]: the current active set
    __shared__ int wsum[16];
    __shared__ int carry_sh, ev_cnt;
    __shared__ int ev_lds[WIN_EVCAP];
    const int tid = threadIdx.x, bd = blockDim.x;
    const int lane = tid & 63, wave = tid >> 6, nw = bd >> 6;
    const int32_t *old = ring + (size_t)head * ff;
    // round trip 1: sizes and state; the first expiring entry (in bounds whatever old_len is)
    const int n_act = min(max(*n_active_p, 0), ff);
    const int old_set = ring_set[head];
    const int old_len0 = ring_len[head];
    const int n_free0 = min(max(state[0], 0), ff), hw = min(max(state[1], 0), ff);
    const int n_res0 = state[2];
    const int o_pre = old[min(tid, ff - 1)];
    const int old_len = old_set ? min(max(old_len0, 0), ff) : 0;
    auto nid = [&](int v) { return v >= 0 && v < ff ? v : -1; };  // an index, or -1
    for (int i = tid; i < (ff + 31) / 32; i += bd) curbits[i] = 0;
    if (tid == 0) {
        carry_sh = 0;
        ev_cnt = 0;
    }
    // round trip 2: first active entry and its slot; first expiring entry's
    // slot and count after the decrement (A, window.go:73-80)
    const int a0 = tid < n_act ? nid(active[tid]) : -1;
    const int sa0 = a0 >= 0 ? slot_of[a0] : 0;
    const int o0 = tid < old_len ? nid(o_pre) : -1;
    // cnt belongs to this one workgroup, so the decrement is a plain load and
    // store (a returning atomic takes a longer round trip)
    int so0 = -1, c0 = 1;
    if (o0 >= 0) {
        so0 = slot_of[o0];
        c0 = cnt[o0] - 1;
        cnt[o0] = c0;
    }
    __syncthreads();
    // B: mark the current set
    if (a0 >= 0) atomicOr(&curbits[a0 >> 5], 1u << (a0 & 31));
    for (int j = tid + bd; j < n_act; j += bd) {
        const int n = nid(active[j]);
        if (n >= 0) atomicOr(&curbits[n >> 5], 1u << (n & 31));
    }
    __syncthreads();
    // C: an expiring neuron no set holds any more is evicted (window.go:84-95).
    // Each entry of the expiring set is one thread's, so its decremented count
    // is final here (the counts of current neurons only grow, in E).
    auto evict = [&](int n, int s, int c) {
        if (c == 0 && !((curbits[n >> 5] >> (n & 31)) & 1u) && s >= 0) {
            slot_of[n] = -1;
            const int e = atomicAdd(&ev_cnt, 1);
            if (n_free0 + e < ff) free_stack[n_free0 + e] = s;
            if (e < WIN_EVCAP) ev_lds[e] = s;
        }
    };
    if (o0 >= 0) evict(o0, so0, c0);
    for (int j = tid + bd; j < old_len; j += bd) {
        const int n = nid(old[j]);
        if (n < 0) continue;
        const int sn = slot_of[n];
        const int c = cnt[n] - 1;
        cnt[n] = c;
        evict(n, sn, c);
    }
    __syncthreads();
    // D: toLoad in active order (window.go:98-103) by a block-wide scan; the
    // k-th needed neuron pops the k-th slot from the top of the free stack
    // (this update's evictions, then the older entries), then fresh slots.
    const int n_ev = min(ev_cnt, ff - n_free0);  // evictions kept on the stack
    const int n_free = n_free0 + n_ev;
    for (int j0 = 0; j0 < n_act; j0 += bd) {
        const int j = j0 + tid;
        int n = -1, need = 0;
        if (j0 == 0) {
            n = a0;
            need = (n >= 0 && sa0 < 0) ? 1 : 0;  // evictions never touch current neurons
        } else if (j < n_act) {
            n = nid(active[j]);
            need = (n >= 0 && slot_of[n] < 0) ? 1 : 0;
        }
        int incl = need;
        for (int o = 1; o < 64; o <<= 1) {
            const int v = __shfl_up(incl, o, 64);
            if (lane >= o) incl += v;
        }
        if (lane == 63) wsum[wave] = incl;
        __syncthreads();
        int before = carry_sh;
        for (int w = 0; w < wave; w++) before += wsum[w];
        int total = carry_sh;
        for (int w = 0; w < nw; w++) total += wsum[w];
        if (need) {
            const int kidx = before + incl - 1;
            int sl;
            if (kidx < n_ev) {
                const int e = n_ev - 1 - kidx;
                sl = e < WIN_EVCAP ? ev_lds[e] : free_stack[n_free0 + e];
            } else if (kidx < n_free) {
                sl = free_stack[n_free - 1 - kidx];
            } else {
                sl = hw + (kidx - n_free);
                if (sl >= ff) sl = -1;  // no room (only a list with repeats gets here)
            }
            slot_of[n] = sl;
            if (sl >= 0) fresh[n] = epoch;
            load_list[2 * kidx] = n;
            load_list[2 * kidx + 1] = sl;
        }
        __syncthreads();
        if (tid == 0) carry_sh = total;
        __syncthreads();
    }
    // E: counts of the current set, the ring slot, the head (window.go:113-114)
    int32_t *dst = ring + (size_t)head * ff;
    if (tid < n_act) dst[tid] = a0;
    if (a0 >= 0) atomicAdd(&cnt[a0], 1);
    for (int j = tid + bd; j < n_act; j += bd) {
        const int n = nid(active[j]);
        if (n >= 0) atomicAdd(&cnt[n], 1);
        dst[j] = n;
    }
    if (tid == 0) {
        const int n_load = carry_sh;
        state[0] = n_load < n_free ? n_free - n_load : 0;
        state[1] = min(ff, hw + (n_load > n_free ? n_load - n_free : 0));
        state[2] = n_res0 - n_ev + n_load;
        state[3] = n_load;
        ring_len[head] = n_act;
        ring_set[head] = 1;
    }
}

// One workgroup per loaded neuron: copy its bundle (bstride bytes, a multiple
// of 128) into its resident slot with 16-byte loads and stores.
__global__ __launch_bounds__(256) void k_window_gather(const uint8_t *__restrict__ src,
                                                       uint8_t *__restrict__ dst,
                                                       long long bstride,
                                                       const int32_t *__restrict__ load_list,
                                                       const int32_t *__restrict__ state) {
    const int n_load = state[3];
    const int n16 = (int)(bstride >> 4);
    for (int i = blockIdx.x; i < n_load; i += gridDim.x) {
        const int n = load_list[2 * i];
        const int s = load_list[2 * i + 1];
        if (s < 0) continue;  // left non-resident (the update found no slot)
        const uint4 *sp = reinterpret_cast<const uint4 *>(src + (long long)n * bstride);
        uint4 *dp = reinterpret_cast<uint4 *>(dst + (long long)s * bstride);
        for (int c = threadIdx.x; c < n16; c += blockDim.x) dp[c] = sp[c];
    }
}

static LlgWindow *get_window(LlgDevice *d, int64_t h) {
    LlgObject *o = llg_get(d, h, LLG_KIND_WINDOW);
    return o ? reinterpret_cast<LlgWindow *>(o->ext) : nullptr;
}

// gather = false: the caller's FFN launch copies the loaded bundles (the
// k_list_up form that reads fresh tags).
static int window_update_enqueue(LlgDevice *d, LlgWindow *w, const int32_t *d_active,
                                 const int32_t *d_n_active, int max_active, bool gather) {
    hipStream_t st = llg_dev_stream(d);
    const size_t bits = (size_t)(w->ff + 31) / 32 * 4;
    w->epoch = w->epoch == 0x7FFFFFFF ? 1 : w->epoch + 1;
    hipLaunchKernelGGL(k_window_update, dim3(1), dim3(1024), bits, st, w->slot_of, w->cnt, w->ring,
                       w->ring_len, w->ring_set, w->free_stack, w->state, w->load_list, w->fresh,
                       w->epoch, d_active, d_n_active, w->head, w->ff);
    LLG_LAUNCH_CHECK(d, "window_update");
    if (gather) {
        int grid = max_active < 1 ? 1 : (max_active > 2048 ? 2048 : max_active);
        hipLaunchKernelGGL(k_window_gather, dim3(grid), dim3(256), 0, st, w->bundle->d,
                           w->resident, w->bstride, w->load_list, w->state);
        LLG_LAUNCH_CHECK(d, "window_gather");
    }
    w->head = (w->head + 1) % w->k;
    return 0;
}

extern "C" {

int llg_hip_window_create(LlgHipDevice h, int64_t hb, int k, int64_t *win) {
    LlgDevice *d = llg_dev(h);
    if (!d) return LLG_E_NODEV;
    LlgObject *b = llg_get(d, hb, LLG_KIND_BUNDLE);
    if (!b) return llg_set_error(d, LLG_E_HANDLE, "window_create: unknown bundle");
    if (k < 1 || !win) return llg_set_error(d, LLG_E_ARG, "window_create: k must be >= 1");
    if ((size_t)(b->rows + 31) / 32 * 4 > 48 * 1024)  // the update's LDS bitmap
        return llg_set_error(d, LLG_E_ARG, "window_create: %d neurons, at most 393216", b->rows);
    LlgWindow *w = new LlgWindow();
    w->bundle = b;
    w->k = k;
    w->ff = b->rows;
    w->head = 0;
    w->cap = b->rows;
    w->bstride = b->stride;
    const size_t ff = (size_t)w->ff;
    // one allocation for the int32 state arrays
    const size_t n_ints = ff * 2 + (size_t)k * ff + 2 * (size_t)k + ff + 4 + 2 * ff + ff;
    int32_t *m = nullptr;
    if (hipMalloc(&m, n_ints * 4) != hipSuccess) {
        delete w;
        return llg_set_error(d, LLG_E_NOMEM, "window_create: state allocation failed");
    }
    w->slot_of = m;
    w->cnt = m + ff;
    w->ring = m + 2 * ff;
    w->ring_len = w->ring + (size_t)k * ff;
    w->ring_set = w->ring_len + k;
    w->free_stack = w->ring_set + k;
    w->state = w->free_stack + ff;
    w->load_list = w->state + 4;
    w->fresh = w->load_list + 2 * ff;  // 0: never loaded (updates are numbered from 1)
    w->epoch = 0;
    if (hipMalloc(&w->resident, (size_t)w->cap * w->bstride) != hipSuccess) {
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
    o->bytes = (size_t)w->cap * w->bstride;
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
                                    n_active, true)))
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
    if ((rc = window_update_enqueue(d, w, d_active, d_n_active, w->ff, false))) return rc;
    const LlgFreshRows fr{w->bundle->d, w->fresh, w->epoch, w->resident};
    return llg_sparse_enqueue(d, w->resident, w->bstride, w->bundle->fmt, w->slot_of, d_x,
                              d_active, d_n_active, w->ff, w->ff, act, d_out, ws, &fr);
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
