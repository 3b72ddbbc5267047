// llg_window_upd.hpp -- the window update (inference/window.go:71-117) split
// over workgroups, shared by the window's plain update (llg_window.hip) and
// its update + FFN step (k_win_step, llg_sparse.hip).  Neuron n lives in row
// n of the resident buffer, so the update needs no slot allocation.  Counts
// are integer atomics, so every result is the same on every run.
#pragma once
#include "llg_common.hpp"
#include "llg_internal.hpp"

// Whether n was resident at the start of update e (the update marks its loads
// with res[n] = e, so a reader of the same launch sees 0 or e for them).
__device__ __forceinline__ bool win_resident(const int32_t *res, int n, int e) {
    const int r = __hip_atomic_load(res + n, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    return r != 0 && r != e;
}

// 32-bit words of the LDS bitmap of the listed set that win_update_part takes.
__host__ __device__ constexpr int win_bitmap_words(int n_rows) { return (n_rows + 31) >> 5; }

// Part `part` of `n_parts` of update e, by one workgroup, from the listed set
// active[0..n_listed) (an index outside [0, n_rows) is recorded as -1 and
// skipped), the expiring set and the state at the start.  bm: LDS room for
// win_bitmap_words(n_rows) words, where every part builds the bitmap of the
// listed set.  Entries j = part, part + n_parts, ... of the set are recorded
// in the ring and counted, and a neuron not resident at the start is marked
// loaded (res = e; one load per entry, as the reference's loadRows takes each
// listed row it misses).  The same entries of the expiring set are uncounted
// (window.go:73-80); the uncount that takes a count to 0 evicts the neuron
// (res = 0, window.go:84-95) unless the listed set holds it, which is the
// reference's stillNeeded test: that count is 0 exactly when none of the
// other k - 1 sets and not the new set holds it, and an uncount of a listed
// neuron never evicts it, however the counts of the parts interleave.  The
// loads are added to cntr[e & 1] (the next update's counter is cleared) and
// the change of the resident count to state[2].
__device__ __forceinline__ void win_update_part(const LlgWinUpd &u, const int32_t *active,
                                                int n_listed, int n_rows, int part, int n_parts,
                                                uint32_t *bm) {
    __shared__ int wu_loads, wu_delta;
    const int tid = threadIdx.x, bd = blockDim.x, e = u.epoch;
    const int nw = win_bitmap_words(n_rows);
    for (int i = tid; i < nw; i += bd) bm[i] = 0u;
    if (tid == 0) {
        wu_loads = 0;
        wu_delta = 0;
    }
    __syncthreads();
    for (int j = tid; j < n_listed; j += bd) {
        const int n = active[j];
        if (n >= 0 && n < n_rows) atomicOr(bm + (n >> 5), 1u << (n & 31));
    }
    __syncthreads();
    int loads = 0, delta = 0;
    for (int j = part + n_parts * tid; j < n_listed; j += n_parts * bd) {
        int n = active[j];
        n = n >= 0 && n < n_rows ? n : -1;
        u.ring_new[j] = n;
        if (n < 0) continue;
        atomicAdd(u.cnt + n, 1);
        if (!win_resident(u.res, n, e)) {
            loads++;
            if (atomicExch(u.res + n, e) == 0) delta++;
        }
    }
    const int len = *u.ring_set_exp ? min(max(*u.ring_len_exp, 0), n_rows) : 0;
    for (int i = part + n_parts * tid; i < len; i += n_parts * bd) {
        const int n = u.ring_exp[i];
        if (n < 0 || n >= n_rows) continue;
        if (atomicSub(u.cnt + n, 1) == 1 && !((bm[n >> 5] >> (n & 31)) & 1u) &&
            atomicExch(u.res + n, 0) != 0)
            delta--;
    }
    if (loads) atomicAdd(&wu_loads, loads);
    if (delta) atomicAdd(&wu_delta, delta);
    __syncthreads();
    if (tid == 0) {
        if (wu_loads) atomicAdd(u.cntr + (e & 1), wu_loads);
        if (wu_delta) atomicAdd(u.state + 2, wu_delta);
        if (part == 0) {
            *u.ring_len_new = n_listed;
            *u.ring_set_new = 1;
            u.cntr[(e + 1) & 1] = 0;
        }
    }
}
