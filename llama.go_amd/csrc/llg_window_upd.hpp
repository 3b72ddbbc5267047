// llg_window_upd.hpp -- the per-entry steps of the window update
// (inference/window.go:71-117) shared by the window's own kernels
// (llg_window.hip) and the list FFN launches of its update + FFN step
// (llg_sparse.hip).  Neuron n lives in row n of the resident buffer, so the
// update needs no slot allocation: each step below touches one neuron, and
// the only ordering is the launch boundary between the first three and the
// last three.  Counts are integer atomics, so every result is the same on
// every run.
#pragma once
#include "llg_common.hpp"
#include "llg_internal.hpp"

// First launch.  Entry j of the listed set (n = -1: absent): recorded in the
// ring, marked and counted; returns whether n must be loaded (it was not
// resident before this update; nothing writes slot_of in this launch).
__device__ __forceinline__ bool win_note_active(const LlgWinUpd &u, int j, int n) {
    u.ring_new[j] = n;
    if (n < 0) return false;
    u.cur_ep[n] = u.epoch;
    atomicAdd(&u.cnt[n], 1);
    return u.slot_of[n] < 0;
}
// ... after its bundle copy is issued: the load is tagged and counted.
__device__ __forceinline__ void win_note_load(const LlgWinUpd &u, int n) {
    u.fresh[n] = u.epoch;
    atomicAdd(&u.cntr[u.epoch & 1], 1);
}
// Entries of the expiring set (window.go:73-80), grid-stride over gt / gs
// threads; one thread also records the new set's length.  n_rows bounds the
// indices (an entry outside [0, n_rows) is skipped).
__device__ __forceinline__ void win_expire_all(const LlgWinUpd &u, int n_listed, int n_rows,
                                               int gt, int gs) {
    const int len = *u.ring_set_exp ? min(max(*u.ring_len_exp, 0), n_rows) : 0;
    for (int i = gt; i < len; i += gs) {
        const int n = u.ring_exp[i];
        if (n >= 0 && n < n_rows) atomicSub(&u.cnt[n], 1);
    }
    if (gt == 0) {
        *u.ring_len_new = n_listed;
        *u.ring_set_new = 1;
    }
}

// Second launch (grid-stride): an expiring neuron that no set holds any more
// is evicted (window.go:84-95); a loaded one becomes resident; one thread
// publishes the load count and clears the next update's counter.  The two
// loops touch disjoint neurons (an evicted one is not listed, a loaded one was
// not resident), and the exchanges count each neuron once.
__device__ __forceinline__ void win_finish_all(const LlgWinUpd &u, int n_listed, int n_rows,
                                               int gt, int gs) {
    const int len = *u.ring_set_exp ? min(max(*u.ring_len_exp, 0), n_rows) : 0;
    for (int i = gt; i < len; i += gs) {
        const int n = u.ring_exp[i];
        if (n >= 0 && n < n_rows && u.cnt[n] == 0 && u.cur_ep[n] != u.epoch &&
            atomicExch(&u.slot_of[n], -1) >= 0)
            atomicSub(&u.state[2], 1);
    }
    for (int j = gt; j < n_listed; j += gs) {
        const int n = u.ring_new[j];
        if (n >= 0 && u.fresh[n] == u.epoch && atomicExch(&u.slot_of[n], n) < 0)
            atomicAdd(&u.state[2], 1);
    }
    if (gt == 0) {
        u.state[3] = u.cntr[u.epoch & 1];
        u.cntr[(u.epoch + 1) & 1] = 0;
    }
}
