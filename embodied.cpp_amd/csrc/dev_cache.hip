// Device-resident LingBot runtime-KV slot metadata, gfx950.
//
// The reference keeps the slot metadata of each (model, session, layer,
// branch) cache on the host (LingBotKVCache, models/lingbot_va.cpp:8740-8997)
// and, per layer and call, scans it under a global mutex, then copies the
// chosen slots and the valid-slot list to the device with synchronous
// cudaMemcpy before the update kernel and the attention run
// (run_lingbot_runtime_kv_device_attention, :9568-9650, called from
// :9697-9767).  Here the metadata (id, mask, is_pred per slot) lives in device
// memory and one single-workgroup kernel per call performs the whole update:
//   * allocate_slots_into (:8793-8831): the free slots in ascending order; if
//     too few, the `need` valid slots with the lowest ids are evicted (mask 0,
//     id -1, and is_pred 0 in the legacy mode), ties between equal ids in
//     ascending slot order, and the evictions stay when the call then fails;
//   * update_meta_only (:8887-8902), modes 1 (prediction) and 2 (clean):
//     new_id = next_id() after the evictions, the chosen slots stamped
//     (mask 1, id, is_pred); the valid list is then collect_valid_slots
//     (:8967-8972);
//   * prepare_mode0_temp_slots_no_insert (:8904-8944), mode 0: the chosen
//     slots get id = next_id() and is_pred 0 but stay invisible (mask 0); the
//     valid list is every visible slot and the chosen ones, ascending.
// The slots, the valid list and its length land in device buffers that the
// append and the attention read directly on the same stream: no host scan,
// no synchronous copy.  restore (:8946-8952) and clear_pred (:8954-8965) are
// elementwise kernels.
//
// One workgroup of 512 threads (8 waves).  Wave w owns the contiguous slot
// range [w*S, (w+1)*S), S a whole number of 64-slot rounds; in round r lane l
// handles slot w*S + 64 r + l.  Every global access is then one coalesced
// 64-slot row, and the ascending-slot ranks inside a wave are ballots and
// mbcnt (lanes below in the same round, plus the earlier rounds' counts).
// Across waves each step exchanges one row of per-wave values through LDS
// with a single barrier, and every thread reads all 8 rows.  The eviction
// threshold T (the id below which every valid slot goes) is the lowest valid
// id when that id alone covers the eviction -- the steady state of a sliding
// window, where the oldest chunk goes -- and otherwise a bisection over the id
// range, one counting pass a step.  For caches of up to 16384 slots the
// metadata of a lane's rounds stays in registers for the whole call (ids as
// they are, the masks as one bit a round).
#include <hip/hip_runtime.h>

#include <climits>

#include "emb_common.h"

namespace {

constexpr int NT = 512;
constexpr int NW = NT / 64;
constexpr int RMAX = 32;                     // rounds held in registers
constexpr int REG_SLOTS = NW * 64 * RMAX;    // 16384

struct DevCache {
    int64_t *id;
    uint8_t *mask;
    uint8_t *is_pred;
    int32_t capacity;
    int32_t legacy;
};

// One row of up to four per-wave values, in two buffers used alternately: an
// exchange's single barrier then also orders it after every thread's reads of
// the other buffer in the exchange before.
struct Rows {
    int64_t v[2][NW][4];
};

__device__ __forceinline__ int32_t lanes_below(uint64_t m) {
    return (int32_t)__builtin_amdgcn_mbcnt_hi((uint32_t)(m >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)m, 0u));
}

// A 64-bit DPP lane move (both halves with the same pattern; every pattern
// used here reads a lane of the same row, so all lanes are written).
template <int CTRL>
__device__ __forceinline__ int64_t dpp64(int64_t v) {
    const uint64_t u = (uint64_t)v;
    const uint32_t lo = (uint32_t)__builtin_amdgcn_update_dpp(0, (int)(uint32_t)u, CTRL, 0xf, 0xf, false);
    const uint32_t hi = (uint32_t)__builtin_amdgcn_update_dpp(0, (int)(uint32_t)(u >> 32), CTRL, 0xf, 0xf, false);
    return (int64_t)(((uint64_t)hi << 32) | lo);
}

__device__ __forceinline__ int64_t lane64(int64_t v, int l) {
    const uint64_t u = (uint64_t)v;
    const uint32_t lo = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)u, l);
    const uint32_t hi = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)(u >> 32), l);
    return (int64_t)(((uint64_t)hi << 32) | lo);
}

// Wave sum of v, uniform (the same lane pattern as wave_ext below).
__device__ __forceinline__ int32_t wave_sum(int32_t v) {
    v += __builtin_amdgcn_update_dpp(0, v, 0xB1, 0xf, 0xf, false);
    v += __builtin_amdgcn_update_dpp(0, v, 0x4E, 0xf, 0xf, false);
    v += __builtin_amdgcn_update_dpp(0, v, 0x141, 0xf, 0xf, false);
    v += __builtin_amdgcn_update_dpp(0, v, 0x140, 0xf, 0xf, false);
    return __builtin_amdgcn_readlane(v, 0) + __builtin_amdgcn_readlane(v, 16) + __builtin_amdgcn_readlane(v, 32) +
           __builtin_amdgcn_readlane(v, 48);
}

// Wave minimum (MAX = false) or maximum of v, uniform: within quads (lane
// xor 1, xor 2), then across the two quads of each 8-lane half (half mirror)
// and the two halves of each 16-lane row (row mirror), then the four rows.
// All 64 lanes must be active.
template <bool MAX>
__device__ __forceinline__ int64_t wave_ext(int64_t v) {
    auto pick = [](int64_t a, int64_t b) { return MAX ? (a > b ? a : b) : (a < b ? a : b); };
    v = pick(v, dpp64<0xB1>(v));   // quad_perm(1, 0, 3, 2)
    v = pick(v, dpp64<0x4E>(v));   // quad_perm(2, 3, 0, 1)
    v = pick(v, dpp64<0x141>(v));  // row_half_mirror
    v = pick(v, dpp64<0x140>(v));  // row_mirror
    return pick(pick(lane64(v, 0), lane64(v, 16)), pick(lane64(v, 32), lane64(v, 48)));
}

// status: 0 = done, EMB_ERR_CAPACITY = too few slots even after evicting every
// valid slot (the evictions persist, as in the reference).
template <bool REG>
__global__ __launch_bounds__(NT) void meta_update_kernel(DevCache c, int32_t key_size, int32_t mode,
                                                         int32_t *__restrict__ slots, int32_t *__restrict__ valid,
                                                         int32_t *__restrict__ n_valid,
                                                         int32_t *__restrict__ status) {
    __shared__ Rows rows;
    int flip = 0;
    const int t = threadIdx.x, lane = t & 63;
    const int w = __builtin_amdgcn_readfirstlane(t >> 6);
    const int32_t cap = c.capacity;
    const int32_t S = ((cap + NW - 1) / NW + 63) / 64 * 64;  // slots a wave owns, whole rounds
    const int32_t nr = S / 64;
    const int32_t w0 = w * S, wend = min(w0 + S, cap);

    // exchange up to four per-wave values; returns the buffer every thread then reads
    auto exchange = [&](int64_t a, int64_t b, int64_t d, int64_t e) __attribute__((always_inline)) {
        int64_t(*buf)[4] = rows.v[flip];
        flip ^= 1;
        if (lane == 0) {
            buf[w][0] = a;
            buf[w][1] = b;
            buf[w][2] = d;
            buf[w][3] = e;
        }
        __syncthreads();
        return buf;
    };

    // f(r, s, present, mask&, id&) for each round in ascending slot order; the
    // whole wave calls f every round (absent lanes with present = false), so f
    // may take ballots.  Not REG: changes of mask / id are stored in place.
    int64_t ri[REG ? RMAX : 1];
    uint32_t mbits = 0;  // REG: bit r = mask of round r's slot (nonzero -> 1)
    uint32_t dirty = 0;  // REG: rounds whose slot this lane changed
    auto each = [&](auto &&f) __attribute__((always_inline)) {
        if constexpr (REG) {
#pragma unroll
            for (int r = 0; r < RMAX; ++r) {
                if (r < nr) {
                    const int32_t s = w0 + r * 64 + lane;
                    uint8_t m = (mbits >> r) & 1u;
                    f(r, s, s < wend, m, ri[r]);
                    mbits = (mbits & ~(1u << r)) | ((uint32_t)(m != 0) << r);
                }
            }
        } else {
            for (int32_t r = 0; r < nr; ++r) {
                const int32_t s = w0 + r * 64 + lane;
                const bool in = s < wend;
                uint8_t m = in ? c.mask[s] : 0;
                int64_t id = in ? c.id[s] : -1;
                const uint8_t m0 = m;
                const int64_t id0 = id;
                f(r, s, in, m, id);
                if (in && (m != m0 || id != id0)) {
                    c.mask[s] = m;
                    c.id[s] = id;
                }
            }
        }
    };
    if constexpr (REG) {
#pragma unroll
        for (int r = 0; r < RMAX; ++r) {
            const int32_t s = w0 + r * 64 + lane;
            const bool in = r < nr && s < wend;
            if (in && c.mask[s]) mbits |= 1u << r;
            ri[r] = in ? c.id[s] : -1;
        }
    }

    // One pass: free count, the id range of the valid slots and how many hold
    // the lowest id (counts kept per lane and summed once: no per-round
    // ballot chain).  A wave's slots in range: its share of [0, cap).
    auto in_range = [&](int i) { return max(0, min(S, cap - i * S)); };
    int32_t nfree = 0, cmn = 0;
    int64_t mn = LLONG_MAX, mx = LLONG_MIN;
    each([&](int, int32_t, bool in, uint8_t &m, int64_t &id) {
        nfree += in && !m;
        if (in && m) {
            cmn = id < mn ? 1 : cmn + (id == mn);
            mn = id < mn ? id : mn;
            mx = id > mx ? id : mx;
        }
    });
    nfree = wave_sum(nfree);
    {
        const int64_t wmn = wave_ext<false>(mn);
        cmn = wave_sum(mn == wmn ? cmn : 0);
        mn = wmn;
    }
    mx = wave_ext<true>(mx);
    int32_t free_total = 0, atmin_total = 0, atmin_before = 0;
    int32_t frank = 0, vrank = 0, nv_total = 0;  // final ranks: this wave's first free / listed rank
    int64_t idmin = LLONG_MAX, idmax = LLONG_MIN;
    // per-wave (free, valid) after the call's evictions -> ranks
    auto ranks = [&](auto &&nf_of, auto &&nv_of) __attribute__((always_inline)) {
        int32_t fbefore = 0;
        nv_total = 0;
#pragma unroll
        for (int i = 0; i < NW; ++i) {
            const int32_t nfi = nf_of(i), nvi = nv_of(i);
            const int32_t chosen = min(max(key_size - fbefore, 0), nfi);
            if (i == w) {
                frank = fbefore;
                vrank = nv_total;
            }
            fbefore += nfi;
            nv_total += nvi + chosen;
        }
    };
    int32_t nfree_of[NW];  // per wave; kept here, the exchange buffer is reused
    {
        int64_t(*b)[4] = exchange(nfree, mn, cmn, mx);
#pragma unroll
        for (int i = 0; i < NW; ++i) {
            nfree_of[i] = (int32_t)b[i][0];
            free_total += nfree_of[i];
            idmin = b[i][1] < idmin ? b[i][1] : idmin;
            idmax = b[i][3] > idmax ? b[i][3] : idmax;
        }
#pragma unroll
        for (int i = 0; i < NW; ++i) {
            const int32_t c_i = b[i][1] == idmin ? (int32_t)b[i][2] : 0;
            atmin_total += c_i;
            atmin_before += i < w ? c_i : 0;
        }
    }
    const int32_t used_total = cap - free_total;
    int32_t used_after = used_total;

    if (free_total < key_size && used_total > 0) {
        // evict the e lowest (id, slot) valid slots: every valid slot with
        // id < T and the first take_at (ascending slot) with id == T
        const int32_t e = min(key_size - free_total, used_total);
        int64_t T = idmin;
        int32_t below_total = 0, at_total = atmin_total, at_before = atmin_before;
        if (at_total < e) {
            // smallest T in (idmin, idmax] with count(valid, id <= T) >= e
            int64_t lo = idmin + 1, hi = idmax;
            while (lo < hi) {
                const int64_t mid = lo + ((hi - lo) >> 1);
                int32_t n = 0;
                each([&](int, int32_t, bool in, uint8_t &m, int64_t &id) { n += in && m && id <= mid; });
                int64_t(*b)[4] = exchange(wave_sum(n), 0, 0, 0);
                int32_t tot = 0;
#pragma unroll
                for (int i = 0; i < NW; ++i) tot += (int32_t)b[i][0];
                if (tot >= e)
                    hi = mid;
                else
                    lo = mid + 1;
            }
            T = lo;
            int32_t below = 0, at = 0;
            each([&](int, int32_t, bool in, uint8_t &m, int64_t &id) {
                below += in && m && id < T;
                at += in && m && id == T;
            });
            int64_t(*b)[4] = exchange(wave_sum(below), wave_sum(at), 0, 0);
            at_total = at_before = 0;
#pragma unroll
            for (int i = 0; i < NW; ++i) {
                below_total += (int32_t)b[i][0];
                at_before += i < w ? (int32_t)b[i][1] : 0;
                at_total += (int32_t)b[i][1];
            }
        }
        const int32_t take_at = e - below_total;
        int32_t nev = 0;
        auto evict = [&](int r, int32_t s, uint8_t &m, int64_t &id) __attribute__((always_inline)) {
            m = 0;
            id = -1;
            dirty |= 1u << r;
            ++nev;
            if (c.legacy) c.is_pred[s] = 0;
        };
        if (take_at >= at_total) {  // the whole id == T group goes (a window's oldest chunk): no ranks
            each([&](int r, int32_t s, bool in, uint8_t &m, int64_t &id) {
                if (in && m && id <= T) evict(r, s, m, id);
            });
        } else {
            int32_t run = at_before;
            each([&](int r, int32_t s, bool in, uint8_t &m, int64_t &id) {
                const bool valid_slot = in && m;
                const uint64_t bm = __ballot(valid_slot && id == T);
                const int32_t rank = run + lanes_below(bm);
                run += (int32_t)__popcll(bm);
                if (valid_slot && (id < T || (id == T && rank < take_at))) evict(r, s, m, id);
            });
        }
        nev = wave_sum(nev);
        free_total += e;
        used_after = used_total - e;
        if (free_total >= key_size) {
            int64_t(*b)[4] = exchange(nev, 0, 0, 0);
            ranks([&](int i) { return nfree_of[i] + (int32_t)b[i][0]; },
                  [&](int i) { return in_range(i) - (nfree_of[i] + (int32_t)b[i][0]); });
        }
    } else if (free_total >= key_size) {
        ranks([&](int i) { return nfree_of[i]; }, [&](int i) { return in_range(i) - nfree_of[i]; });
    }
    const bool ok = free_total >= key_size;
    if (ok) {
        // new_id = next_id() after the evictions, before the stamps.  Evictions
        // take the lowest ids first, so a valid slot that remains leaves idmax
        // the largest id; none remaining leaves next_id() = 0.
        const int64_t new_id = used_after > 0 ? idmax + 1 : 0;
        // chosen: the first key_size free slots in ascending order; listed
        // after the call: the visible ones and the chosen ones (which modes 1/2
        // make visible and mode 0 lists as temporaries).  When every slot ends
        // up listed (a full window) the list is 0 .. cap-1 and needs no ranks.
        const bool all_listed = nv_total == cap;
        auto stamp = [&](int r, int32_t s, bool in, uint8_t &m, int64_t &id) __attribute__((always_inline)) {
            const bool fre = in && !m;
            const uint64_t fm = __ballot(fre);
            const int32_t fr = frank + lanes_below(fm);
            frank += (int32_t)__popcll(fm);
            const bool chosen = fre && fr < key_size;
            const bool listed = (in && m) || chosen;
            if (chosen) {
                slots[fr] = s;
                id = new_id;
                c.is_pred[s] = mode == 1;
                if (mode != 0) m = 1;
                dirty |= 1u << r;
            }
            return listed;
        };
        if (all_listed || !valid) {
            each([&](int r, int32_t s, bool in, uint8_t &m, int64_t &id) {
                stamp(r, s, in, m, id);
                if (valid && in) valid[s] = s;
            });
        } else {
            each([&](int r, int32_t s, bool in, uint8_t &m, int64_t &id) {
                const bool listed = stamp(r, s, in, m, id);
                const uint64_t lm = __ballot(listed);
                if (listed) valid[vrank + lanes_below(lm)] = s;
                vrank += (int32_t)__popcll(lm);
            });
        }
        if (t == 0 && n_valid) n_valid[0] = nv_total;
    }
    if constexpr (REG) {  // write back the changed slots (evictions persist on failure too)
#pragma unroll
        for (int r = 0; r < RMAX; ++r) {
            if ((dirty >> r) & 1u) {
                const int32_t s = w0 + r * 64 + lane;
                c.id[s] = ri[r];
                c.mask[s] = (uint8_t)((mbits >> r) & 1u);
            }
        }
    }
    if (!ok) {
        // downstream launches on this stream (append, attention) must see no
        // keys rather than the previous call's lists: every slot -1 (skipped
        // by the append), no valid slot
        for (int32_t i = t; i < key_size; i += NT) slots[i] = -1;
        if (t == 0 && n_valid) n_valid[0] = 0;
    }
    if (t == 0) status[0] = ok ? EMB_OK : EMB_ERR_CAPACITY;
}

__global__ __launch_bounds__(256) void meta_init_kernel(DevCache c) {
    for (int32_t s = blockIdx.x * blockDim.x + threadIdx.x; s < c.capacity; s += gridDim.x * blockDim.x) {
        c.id[s] = -1;
        c.mask[s] = 0;
        c.is_pred[s] = 0;
    }
}

__global__ __launch_bounds__(256) void meta_restore_kernel(DevCache c, const int32_t *__restrict__ slots, int32_t n) {
    for (int32_t i = blockIdx.x * blockDim.x + threadIdx.x; i < n; i += gridDim.x * blockDim.x) {
        const int32_t s = slots[i];
        if (s >= 0 && s < c.capacity) c.mask[s] = 0;
    }
}

__global__ __launch_bounds__(256) void meta_clear_pred_kernel(DevCache c) {
    for (int32_t s = blockIdx.x * blockDim.x + threadIdx.x; s < c.capacity; s += gridDim.x * blockDim.x) {
        if (c.is_pred[s]) {
            c.mask[s] = 0;
            if (c.legacy) {
                c.is_pred[s] = 0;
                c.id[s] = -1;
            }
        }
    }
}

int check_cache(const emb_dev_slot_cache *c) {
    EMB_CHECK_ARG(c && c->id && c->mask && c->is_pred, "null device cache");
    EMB_CHECK_ARG(c->capacity > 0, "capacity must be positive");
    EMB_CHECK_ARG(((uintptr_t)c->id & 7u) == 0, "id must be 8-byte aligned");
    return EMB_OK;
}

DevCache dev(const emb_dev_slot_cache *c) {
    return DevCache{c->id, c->mask, c->is_pred, c->capacity, c->legacy_clear_pred ? 1 : 0};
}

int launched(const char *what) {
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) return emb::set_error(EMB_ERR_LAUNCH, "%s: %s", what, hipGetErrorString(e));
    return EMB_OK;
}

int grid_for(int64_t n) {
    const int64_t g = (n + 255) / 256;
    return (int)(g < 1 ? 1 : (g > 4096 ? 4096 : g));
}

}  // namespace

extern "C" {

int emb_dev_cache_init(const emb_dev_slot_cache *c, hipStream_t stream) {
    if (int rc = check_cache(c)) return rc;
    hipLaunchKernelGGL(meta_init_kernel, dim3(grid_for(c->capacity)), dim3(256), 0, stream, dev(c));
    return launched("emb_dev_cache_init");
}

int emb_dev_cache_update(const emb_dev_slot_cache *c, int32_t key_size, int32_t mode, int32_t *slots,
                         int32_t *valid, int32_t *n_valid, int32_t *status, hipStream_t stream) {
    if (int rc = check_cache(c)) return rc;
    EMB_CHECK_ARG(key_size > 0, "key_size must be positive");
    EMB_CHECK_ARG(mode >= 0 && mode <= 2, "mode must be 0, 1 or 2");
    EMB_CHECK_ARG(slots && status, "null slots / status");
    if (c->capacity <= REG_SLOTS)
        hipLaunchKernelGGL(meta_update_kernel<true>, dim3(1), dim3(NT), 0, stream, dev(c), key_size, mode, slots, valid,
                           n_valid, status);
    else
        hipLaunchKernelGGL(meta_update_kernel<false>, dim3(1), dim3(NT), 0, stream, dev(c), key_size, mode, slots,
                           valid, n_valid, status);
    if (int rc = launched("emb_dev_cache_update")) return rc;
    // Evicting every visible slot frees the whole cache, so the call fails
    // exactly when key_size > capacity: known here, without waiting for the
    // device.  (The kernel still ran: the evictions persist, as in
    // allocate_slots_into, and it wrote slots -1 and n_valid 0.)
    if (key_size > c->capacity)
        return emb::set_error(EMB_ERR_CAPACITY, "key_size %d exceeds the cache capacity %d", key_size, c->capacity);
    return EMB_OK;
}

int emb_dev_cache_restore(const emb_dev_slot_cache *c, const int32_t *slots, int32_t n, hipStream_t stream) {
    if (int rc = check_cache(c)) return rc;
    EMB_CHECK_ARG(slots && n > 0, "null slots or non-positive count");
    hipLaunchKernelGGL(meta_restore_kernel, dim3(grid_for(n)), dim3(256), 0, stream, dev(c), slots, n);
    return launched("emb_dev_cache_restore");
}

int emb_dev_cache_clear_pred(const emb_dev_slot_cache *c, hipStream_t stream) {
    if (int rc = check_cache(c)) return rc;
    hipLaunchKernelGGL(meta_clear_pred_kernel, dim3(grid_for(c->capacity)), dim3(256), 0, stream, dev(c));
    return launched("emb_dev_cache_clear_pred");
}

}  // extern "C"
