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
// One workgroup of 1024 threads; thread i owns the contiguous slot range
// [i*R, (i+1)*R), R = ceil(capacity / 1024), so ascending-slot compaction is a
// per-thread count, one exclusive scan (lane shuffles inside each wave, the 16
// wave totals through LDS) and a per-thread write.  The eviction threshold
// (the id below which every valid slot goes) is found by a bisection over the
// id range of the valid slots, one counting pass a step.  For caches of up to
// 14336 slots each thread's 14 slots stay in registers for the whole call
// (staged through LDS with coalesced loads and written back the same way), so
// the passes never wait on memory.
#include <hip/hip_runtime.h>

#include <climits>

#include "emb_common.h"

namespace {

constexpr int NT = 1024;
constexpr int NW = NT / 64;
// Caches up to this many slots are staged in LDS (8-byte id + 1-byte mask a
// slot, 126 KB at the config-3 capacity of 14040), larger ones are read in place.
constexpr int LDS_SLOTS = 14336;
static_assert(LDS_SLOTS % NT == 0, "whole staging rounds");

struct DevCache {
    int64_t *id;
    uint8_t *mask;
    uint8_t *is_pred;
    int32_t capacity;
    int32_t legacy;
};

// Wave totals of the block reductions, in two buffers used alternately: a
// reduction's single barrier then also orders it after the previous one's
// reads of the other buffer.
struct Scratch {
    int64_t w64[2][NW][2];
    int32_t w32[2][NW];
    int flip;
};

// Exclusive prefix of v over the workgroup (threads in order) and the total:
// an inclusive scan inside each wave by lane shuffles, then the 16 wave totals
// through LDS.  One barrier.
__device__ __forceinline__ int32_t block_scan(int32_t v, Scratch &sc, int &flip, int32_t *total) {
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    int32_t x = v;
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) {
        const int32_t y = __shfl_up(x, off, 64);
        if (lane >= off) x += y;
    }
    int32_t *buf = sc.w32[flip];
    flip ^= 1;
    if (lane == 63) buf[w] = x;
    __syncthreads();
    int32_t before = 0, all = 0;
#pragma unroll
    for (int i = 0; i < NW; ++i) {
        const int32_t a = buf[i];
        before += i < w ? a : 0;
        all += a;
    }
    *total = all;
    return before + x - v;
}

__device__ __forceinline__ int32_t block_sum(int32_t v, Scratch &sc, int &flip) {
    int32_t total;
    block_scan(v, sc, flip, &total);
    return total;
}

// (max a, max b) over the workgroup.  One barrier.
__device__ __forceinline__ void block_max2(int64_t &a, int64_t &b, Scratch &sc, int &flip) {
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) {
        const int64_t ya = __shfl_xor(a, off, 64), yb = __shfl_xor(b, off, 64);
        a = ya > a ? ya : a;
        b = yb > b ? yb : b;
    }
    int64_t(*buf)[2] = sc.w64[flip];
    flip ^= 1;
    if (lane == 0) {
        buf[w][0] = a;
        buf[w][1] = b;
    }
    __syncthreads();
#pragma unroll
    for (int i = 0; i < NW; ++i) {
        a = buf[i][0] > a ? buf[i][0] : a;
        b = buf[i][1] > b ? buf[i][1] : b;
    }
}

// The slots a thread owns, [s0, s0 + n), and their (mask, id).  REG: at
// most PER slots, held in registers for the whole call (staged through LDS
// with coalesced loads; the slots a call changes are stored back), so every
// pass below is register arithmetic.  Otherwise the passes read and write global memory in
// place (caches past LDS_SLOTS).
constexpr int PER = LDS_SLOTS / NT;

template <bool REG>
struct Own {
    int32_t s0, n;
    uint8_t *gm;
    int64_t *gi;
    uint8_t rm[REG ? PER : 1];
    int64_t ri[REG ? PER : 1];

    // f(i, s, mask&, id&) for each owned slot in ascending order
    template <typename F>
    __device__ __forceinline__ void each(F &&f) {
        if constexpr (REG) {
#pragma unroll
            for (int i = 0; i < PER; ++i)
                if (i < n) f(i, s0 + i, rm[i], ri[i]);
        } else {
            for (int32_t i = 0; i < n; ++i) f(i, s0 + i, gm[s0 + i], gi[s0 + i]);
        }
    }
};

// status: 0 = done, EMB_ERR_CAPACITY = too few slots even after evicting every
// valid slot (the evictions persist, as in the reference).
template <bool REG>
__global__ __launch_bounds__(NT) void meta_update_kernel(DevCache c, int32_t key_size, int32_t mode,
                                                         int32_t *__restrict__ slots, int32_t *__restrict__ valid,
                                                         int32_t *__restrict__ n_valid,
                                                         int32_t *__restrict__ status) {
    __shared__ Scratch sc;
    int flip = 0;
    __shared__ int64_t lid[REG ? LDS_SLOTS : 1];
    __shared__ uint8_t lmask[REG ? LDS_SLOTS : 1];
    const int t = threadIdx.x;
    const int32_t R = (c.capacity + NT - 1) / NT;
    Own<REG> own;
    own.s0 = min(t * R, c.capacity);
    own.n = min(own.s0 + R, c.capacity) - own.s0;
    own.gm = c.mask;
    own.gi = c.id;
    uint32_t dirty = 0;  // REG: owned slots this call changed (bit i = slot s0 + i)
    if constexpr (REG) {  // coalesced loads into LDS, then each thread's range into registers
#pragma unroll
        for (int j = 0; j < PER; ++j) {
            const int32_t s = t + j * NT;
            if (s < c.capacity) {
                lid[s] = c.id[s];
                lmask[s] = c.mask[s];
            }
        }
        __syncthreads();
#pragma unroll
        for (int i = 0; i < PER; ++i) {
            own.rm[i] = i < own.n ? lmask[own.s0 + i] : 0;
            own.ri[i] = i < own.n ? lid[own.s0 + i] : 0;
        }
    }

    // free count and the id range of the valid slots
    int32_t nfree = 0;
    int64_t idmin = LLONG_MAX, idmax = LLONG_MIN;
    own.each([&](int, int32_t, uint8_t &m, int64_t &id) {
        if (!m) {
            ++nfree;
        } else {
            idmin = id < idmin ? id : idmin;
            idmax = id > idmax ? id : idmax;
        }
    });
    int32_t free_total = block_sum(nfree, sc, flip);
    const int32_t used_total = c.capacity - free_total;
    bool ok = true;

    if (free_total < key_size && used_total > 0) {
        // evict the e lowest (id, slot) valid slots
        const int32_t e = min(key_size - free_total, used_total);
        int64_t lo = -idmin, hi = idmax;
        block_max2(lo, hi, sc, flip);
        lo = -lo;
        // smallest T with count(valid, id <= T) >= e
        while (lo < hi) {
            const int64_t mid = lo + ((hi - lo) >> 1);
            int32_t n = 0;
            own.each([&](int, int32_t, uint8_t &m, int64_t &id) { n += m && id <= mid; });
            if (block_sum(n, sc, flip) >= e)
                hi = mid;
            else
                lo = mid + 1;
        }
        const int64_t T = lo;
        int32_t below = 0, at = 0;
        own.each([&](int, int32_t, uint8_t &m, int64_t &id) {
            if (m) {
                below += id < T;
                at += id == T;
            }
        });
        const int32_t below_total = block_sum(below, sc, flip);
        int32_t at_total;
        int32_t rank = block_scan(at, sc, flip, &at_total);  // ascending slot order among id == T
        const int32_t take_at = e - below_total;
        own.each([&](int i, int32_t s, uint8_t &m, int64_t &id) {
            if (!m) return;
            bool ev = id < T;
            if (id == T) ev = rank++ < take_at;
            if (ev) {
                m = 0;
                id = -1;
                dirty |= 1u << i;
                if (c.legacy) c.is_pred[s] = 0;
            }
        });
        free_total += e;
    }
    if (free_total < key_size) {
        ok = false;
    } else {
        // new_id = next_id() after the evictions, before the stamps; the first
        // key_size free slots in ascending order
        int32_t nf = 0;
        int64_t mx = -1;
        own.each([&](int, int32_t, uint8_t &m, int64_t &id) {
            if (!m)
                ++nf;
            else
                mx = id > mx ? id : mx;
        });
        int64_t unused64 = 0;
        block_max2(mx, unused64, sc, flip);
        const int64_t new_id = mx + 1;
        int32_t unused;
        int32_t frank = block_scan(nf, sc, flip, &unused);  // free rank of this range's first free slot
        // slots listed after the call: the visible ones and the chosen ones
        // (which modes 1/2 make visible and mode 0 lists as temporaries); the
        // chosen ones of this range are its free slots of rank below key_size
        const int32_t nchosen = min(max(key_size - frank, 0), nf);
        int32_t nv_total;
        int32_t vrank = block_scan(own.n - nf + nchosen, sc, flip, &nv_total);
        own.each([&](int i, int32_t s, uint8_t &m, int64_t &id) {
            bool listed = m != 0;
            if (!listed) {
                if (frank < key_size) {
                    slots[frank] = s;
                    dirty |= 1u << i;
                    id = new_id;
                    c.is_pred[s] = mode == 1;
                    if (mode != 0) m = 1;
                    listed = true;
                }
                ++frank;
            }
            if (valid && listed) valid[vrank++] = s;
        });
        if (t == 0 && n_valid) n_valid[0] = nv_total;
    }
    if constexpr (REG) {  // write back the changed slots (evictions persist on failure too)
#pragma unroll
        for (int i = 0; i < PER; ++i) {
            if ((dirty >> i) & 1u) {
                c.id[own.s0 + i] = own.ri[i];
                c.mask[own.s0 + i] = own.rm[i];
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
    if (c->capacity <= LDS_SLOTS)
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
