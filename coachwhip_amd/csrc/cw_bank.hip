// Expert banks on the device, managed from the host: one layer's n_slots slots of each expert
// matrix, the device expert -> slot table, the LRU bookkeeping (cw_slots) and the host memory
// the experts are copied from.
//
// The reference keeps a layer's bank in Metal shared memory and reads misses from the SSD
// straight into it (ExpertStore::ensure, crates/engine/src/experts.rs:1489-1641; make_bank
// 1320-1378), with the GPU's copy of the table written through shared-memory atomics
// (gpu_sync.rs:70-148, sync_table experts.rs:73-81). On a discrete GPU the slots are HBM and the
// expert store is host memory, so here:
//  - a layer's misses are copied by one kernel on the caller's stream, ordered before the
//    layer's kernels, that reads the host store through its device mapping (pinned memory):
//    one launch moves every miss over PCIe at the rate of a plain DMA copy, where a DMA copy
//    per expert matrix (27 for ten picks) reached under a third of it and cost ~4 µs of host
//    time each. A store without a device mapping (pageable memory) is copied by DMA;
//  - a prefetch (experts.rs:1004-1098) first takes its victims out of the device table on the
//    last ensure's stream (the reference marks the slot not ready and syncs the GPU table before
//    it copies, experts.rs:1052-1058), then copies on the bank's own stream after the work queued
//    on that stream up to the prefetch call (so it overwrites no slot a queued kernel may read),
//    and records an event per slot; ensure waits for that event on its stream (a GPU-side wait,
//    where the reference spins on the host), and a slot still being filled is neither a victim
//    nor listed in the device table;
//  - a matrix the source marks for shrinking (Q3_K, Q4_K or Q5_K in the store) is held as Q2_K:
//    its misses go into a staging area first and are shrunk from there into their slots
//    (ExpertStore::shrink_into, experts.rs:1245-1273), in chunks of STAGE experts; ensure and
//    prefetch each have their own staging area, as they run on different streams;
//  - the device table is patched in stream order by a small kernel whose (expert, slot) pairs
//    travel as kernel arguments, so no host buffer has to outlive the call and nothing here is
//    a memset (the form that stays correct when the caller captures the stream in a graph).
#include <algorithm>
#include <new>
#include <unordered_set>
#include <vector>

#include "cw_common.h"
#include "cw_requant.h"

namespace cw {
namespace {

constexpr int PATCH = 62;  // table entries per patch launch (500-byte argument block)

struct TablePatch {
    uint32_t n;
    uint32_t expert[PATCH];
    uint32_t slot[PATCH];
};

__global__ __launch_bounds__(64) void k_table_patch(uint32_t *table, TablePatch p) {
    const uint32_t i = threadIdx.x;
    if (i < p.n) table[p.expert[i]] = p.slot[i];
}

constexpr int FILL = 64;  // misses per fill launch

constexpr int STAGE = 8;  // experts per staging area (matrices that are shrunk on arrival)

struct FillList {
    const uint8_t *src[3];  // device view of the host store of each matrix
    uint8_t *dst[3];        // the bank's slots of each matrix, or its staging area
    int64_t bytes[3];       // one expert's matrix in the store (a multiple of 16)
    uint32_t staged;        // bit m: matrix m goes to staging position i, not to slot[i]
    uint32_t n;
    uint32_t expert[FILL], slot[FILL];
};

// block (x, y): y = miss * 3 + matrix, x strides that piece's 16-byte words
__global__ __launch_bounds__(256) void k_bank_fill(FillList f) {
    typedef uint32_t v4 __attribute__((ext_vector_type(4)));
    const uint32_t i = blockIdx.y / 3, m = blockIdx.y - 3 * i;
    if (i >= f.n) return;
    const int64_t eb = f.bytes[m];
    const v4 *s = (const v4 *)(f.src[m] + (int64_t)f.expert[i] * eb);
    v4 *d = (v4 *)(f.dst[m] + (int64_t)((f.staged >> m) & 1 ? i : f.slot[i]) * eb);
    const int64_t words = eb / 16;
    for (int64_t j = (int64_t)blockIdx.x * 256 + threadIdx.x; j < words; j += (int64_t)gridDim.x * 256) d[j] = s[j];
}

__global__ __launch_bounds__(256) void k_table_clear(uint32_t *table, int n) {
    const int i = blockIdx.x * 256 + threadIdx.x;
    if (i < n) table[i] = CW_NO_SLOT;
}

size_t align256(size_t x) { return (x + 255) & ~(size_t)255; }

// bytes of one expert's matrix m in a slot: Q2_K when it is shrunk on arrival
int64_t slot_bytes(const cw_bank_source *src, int m) {
    return src->shrink[m] ? src->rows[m] * (src->cols[m] / 256) * 84 : src->expert_bytes[m];
}

int check_source(const cw_bank_source *src, int n_slots) {
    CW_REQUIRE(src, "bank: no source");
    CW_REQUIRE(n_slots > 0 && src->n_experts > 0, "bank: %d slots for %d experts", n_slots, src->n_experts);
    for (int m = 0; m < 3; m++) {
        const int dt = src->dtype[m];
        if (src->shrink[m])
            CW_REQUIRE(dt == CW_Q3_K || dt == CW_Q4_K || dt == CW_Q5_K, "bank: matrix %d of type %d cannot be shrunk", m, dt);
        else
            CW_REQUIRE(is_weight_type(dt), "bank: matrix %d has type %d", m, dt);
        CW_REQUIRE(src->shrink[m] || !src->shape[m], "bank: matrix %d has column weights but is not shrunk", m);
        const int64_t rows = src->rows[m], cols = src->cols[m], bs = cw_block_size(dt);
        CW_REQUIRE(rows > 0 && cols > 0 && cols % bs == 0, "bank: matrix %d is %lld x %lld", m, (long long)rows,
                   (long long)cols);
        const int64_t bytes = rows * (cols / bs) * cw_type_size(dt);
        CW_REQUIRE(src->expert_bytes[m] == bytes, "bank: matrix %d expert is %lld bytes, expected %lld", m,
                   (long long)src->expert_bytes[m], (long long)bytes);
        CW_REQUIRE(src->host[m], "bank: matrix %d has no host source", m);
    }
    return CW_OK;
}

}  // namespace
}  // namespace cw

struct cw_bank {
    int device = -1;
    cw_bank_source src{};
    int n_slots = 0;
    uint8_t *mat[3] = {};
    int64_t slot_eb[3] = {};        // one expert's matrix in a slot
    uint8_t *stage[2][3] = {};      // staging of shrunk matrices: [0] ensure, [1] prefetch
    bool any_shrink = false;
    const uint8_t *mapped[3] = {};  // device view of the host store, when it has one
    bool by_kernel = false;         // misses copied by k_bank_fill (else by DMA)
    uint32_t *table = nullptr;
    cw_slots *slots = nullptr;
    std::vector<uint32_t> dev_table;  // the device table once the patches enqueued so far ran
    hipStream_t copy = nullptr;       // prefetch copies
    std::vector<hipEvent_t> slot_ev;  // per slot: end of its last prefetch copy
    std::vector<uint8_t> filling;     // per slot: that copy may still be running
    std::vector<uint8_t> kept;        // per slot: placed by the last ensure
    hipEvent_t fence = nullptr;       // the last ensure's stream, when a prefetch was last called
    hipEvent_t handoff = nullptr;     // the last ensure's stream, when an ensure comes on another one
    hipStream_t last = nullptr;       // the stream of the last ensure
    bool fenced = false;              // an ensure has run (last is set)
    cw_bank_stats st{};

    ~cw_bank() {  // teardown: failures here have no caller to go to
        if (copy) (void)hipStreamSynchronize(copy);
        for (hipEvent_t e : slot_ev)
            if (e) (void)hipEventDestroy(e);
        if (fence) (void)hipEventDestroy(fence);
        if (handoff) (void)hipEventDestroy(handoff);
        if (copy) (void)hipStreamDestroy(copy);
        cw_slots_free(slots);
    }

    int64_t expert_bytes() const { return src.expert_bytes[0] + src.expert_bytes[1] + src.expert_bytes[2]; }  // in the store

    int on_device() const {
        int dev = -1;
        if (hipGetDevice(&dev) != hipSuccess || dev != device)
            return cw::set_error(CW_EINVAL, "bank: made on device %d, called on device %d", device, dev);
        return CW_OK;
    }

    // slots whose prefetch copy has finished stop filling
    int refresh() {
        for (int s = 0; s < n_slots; s++) {
            if (!filling[(size_t)s]) continue;
            const hipError_t q = hipEventQuery(slot_ev[(size_t)s]);
            if (q == hipSuccess) filling[(size_t)s] = 0;
            else if (q != hipErrorNotReady) return cw::set_error(CW_EHIP, "bank: event query: %s", hipGetErrorString(q));
        }
        return CW_OK;
    }

    // copies experts pairs[2i] into slots pairs[2i + 1], i < n, on stream s; matrices that are
    // shrunk pass through staging area `which` (0 for ensure, 1 for prefetch)
    int copy_in(const uint32_t *pairs, int n, hipStream_t s, int which) {
        const int chunk = any_shrink ? cw::STAGE : cw::FILL;
        for (int i0 = 0; i0 < n; i0 += chunk) {
            const int c = std::min(chunk, n - i0);
            if (by_kernel) {
                cw::FillList f{};
                for (int m = 0; m < 3; m++) {
                    f.src[m] = mapped[m];
                    f.dst[m] = src.shrink[m] ? stage[which][m] : mat[m];
                    f.bytes[m] = src.expert_bytes[m];
                    f.staged |= src.shrink[m] ? 1u << m : 0u;
                }
                f.n = (uint32_t)c;
                for (int i = 0; i < c; i++) {
                    f.expert[i] = pairs[2 * (i0 + i)];
                    f.slot[i] = pairs[2 * (i0 + i) + 1];
                }
                // about a thousand blocks in all: enough 16-byte reads in flight to cover PCIe latency
                const int per_piece = std::max(4, std::min(64, (1024 + 3 * c - 1) / (3 * c)));
                hipLaunchKernelGGL(cw::k_bank_fill, dim3(per_piece, 3 * c), dim3(256), 0, s, f);
                if (int rc = cw::check_launch("k_bank_fill")) return rc;
            } else {
                for (int i = 0; i < c; i++)
                    if (int rc = dma(pairs[2 * (i0 + i)], pairs[2 * (i0 + i) + 1], i, s, which)) return rc;
            }
            if (!any_shrink) continue;
            cw::ShrinkIndex idx{};
            for (int i = 0; i < c; i++) idx.i[i] = pairs[2 * (i0 + i) + 1];
            for (int m = 0; m < 3; m++) {
                if (!src.shrink[m]) continue;
                const int64_t bpr = src.cols[m] / 256;
                if (int rc = cw::shrink_pieces(src.dtype[m], stage[which][m], src.expert_bytes[m], idx, c, mat[m], slot_eb[m],
                                               src.rows[m] * bpr, src.shape[m], bpr, s))
                    return rc;
            }
        }
        return CW_OK;
    }

    // DMA copies of expert e: to its slot, or to staging position i for a shrunk matrix
    int dma(uint32_t e, uint32_t slot, int i, hipStream_t s, int which) {
        for (int m = 0; m < 3; m++) {
            const int64_t eb = src.expert_bytes[m];
            uint8_t *dst = src.shrink[m] ? stage[which][m] + (int64_t)i * eb : mat[m] + (int64_t)slot * eb;
            const hipError_t r = hipMemcpyAsync(dst, (const uint8_t *)src.host[m] + (int64_t)e * eb, (size_t)eb,
                                                hipMemcpyHostToDevice, s);
            if (r != hipSuccess) return cw::set_error(CW_EHIP, "bank: copy of expert %u: %s", e, hipGetErrorString(r));
        }
        return CW_OK;
    }

    // brings the device table to the bookkeeping's, leaving out slots still being filled unless
    // the stream has waited for them (listed in waited)
    int publish(const std::vector<uint8_t> &waited, hipStream_t s) {
        std::vector<uint32_t> want((size_t)src.n_experts);
        cw_slots_table(slots, want.data(), src.n_experts);
        cw::TablePatch p{};
        for (int e = 0; e < src.n_experts; e++) {
            uint32_t v = want[(size_t)e];
            if (v != CW_NO_SLOT && filling[v] && !waited[v]) v = CW_NO_SLOT;
            if (v == dev_table[(size_t)e]) continue;
            dev_table[(size_t)e] = v;
            p.expert[p.n] = (uint32_t)e;
            p.slot[p.n] = v;
            if (++p.n == cw::PATCH) {
                hipLaunchKernelGGL(cw::k_table_patch, dim3(1), dim3(64), 0, s, table, p);
                p.n = 0;
            }
        }
        if (p.n) hipLaunchKernelGGL(cw::k_table_patch, dim3(1), dim3(64), 0, s, table, p);
        return cw::check_launch("k_table_patch");
    }
};

extern "C" {

size_t cw_bank_device_bytes(const cw_bank_source *src, int n_slots) {
    if (cw::check_source(src, n_slots) != CW_OK) return 0;
    size_t total = 0;
    for (int m = 0; m < 3; m++) {
        total += cw::align256((size_t)cw::slot_bytes(src, m) * (size_t)n_slots);
        if (src->shrink[m]) total += 2 * cw::align256((size_t)src->expert_bytes[m] * cw::STAGE);
    }
    return total + cw::align256((size_t)src->n_experts * 4);
}

cw_bank *cw_bank_new(const cw_bank_source *src, int n_slots, void *device_mem, size_t bytes) {
    if (cw::check_source(src, n_slots) != CW_OK) return nullptr;
    const size_t need = cw_bank_device_bytes(src, n_slots);
    if (!device_mem || ((uintptr_t)device_mem & 255u) || bytes < need) {
        cw::set_error(CW_EINVAL, "bank: device memory %p of %zu bytes (%zu bytes, 256-byte aligned, needed)", device_mem,
                      bytes, need);
        return nullptr;
    }
    cw_bank *b = new (std::nothrow) cw_bank();
    if (!b) {
        cw::set_error(CW_EINVAL, "bank: out of host memory");
        return nullptr;
    }
    b->src = *src;
    b->n_slots = n_slots;
    b->slots = cw_slots_new(n_slots);
    b->dev_table.assign((size_t)src->n_experts, CW_NO_SLOT);
    b->slot_ev.assign((size_t)n_slots, nullptr);
    b->filling.assign((size_t)n_slots, 0);
    b->kept.assign((size_t)n_slots, 0);
    uint8_t *p = (uint8_t *)device_mem;
    for (int m = 0; m < 3; m++) {
        b->slot_eb[m] = cw::slot_bytes(src, m);
        b->mat[m] = p;
        p += cw::align256((size_t)b->slot_eb[m] * (size_t)n_slots);
        if (src->shrink[m]) {
            b->any_shrink = true;
            for (int w = 0; w < 2; w++) {
                b->stage[w][m] = p;
                p += cw::align256((size_t)src->expert_bytes[m] * cw::STAGE);
            }
        }
    }
    b->table = (uint32_t *)p;
    hipError_t r = hipGetDevice(&b->device);
    // the caller's memory may still be in use by work queued before this call
    if (r == hipSuccess) r = hipDeviceSynchronize();
    if (r == hipSuccess) r = hipStreamCreateWithFlags(&b->copy, hipStreamNonBlocking);
    for (int s = 0; s < n_slots && r == hipSuccess; s++) r = hipEventCreateWithFlags(&b->slot_ev[(size_t)s], hipEventDisableTiming);
    if (r == hipSuccess) r = hipEventCreateWithFlags(&b->fence, hipEventDisableTiming);
    if (r == hipSuccess) r = hipEventCreateWithFlags(&b->handoff, hipEventDisableTiming);
    // the fill kernel needs a device view of all three stores and 16-byte pieces
    b->by_kernel = r == hipSuccess;
    for (int m = 0; m < 3 && b->by_kernel; m++) {
        void *dp = nullptr;
        b->by_kernel = hipHostGetDevicePointer(&dp, const_cast<void *>(src->host[m]), 0) == hipSuccess &&
                       ((uintptr_t)dp & 15u) == 0 && src->expert_bytes[m] % 16 == 0;
        b->mapped[m] = (const uint8_t *)dp;
    }
    (void)hipGetLastError();  // a store without a device view leaves an error behind
    if (r == hipSuccess) {
        hipLaunchKernelGGL(cw::k_table_clear, dim3((src->n_experts + 255) / 256), dim3(256), 0, b->copy, b->table,
                           src->n_experts);
        r = hipGetLastError();
    }
    if (r == hipSuccess) r = hipStreamSynchronize(b->copy);
    if (r != hipSuccess || !b->slots) {
        cw::set_error(r != hipSuccess ? CW_EHIP : CW_EINVAL, "bank: set-up failed: %s", hipGetErrorString(r));
        delete b;
        return nullptr;
    }
    return b;
}

void cw_bank_free(cw_bank *b) { delete b; }

int cw_bank_ensure(cw_bank *b, const uint32_t *needed, int n_needed, cw_stream_t stream, int *n_loaded) {
    if (n_loaded) *n_loaded = 0;
    CW_REQUIRE(b && n_needed >= 0 && (n_needed == 0 || needed), "bank ensure: bad arguments");
    if (int rc = b->on_device()) return rc;
    std::vector<uint32_t> want;
    want.reserve((size_t)n_needed);
    std::unordered_set<uint32_t> seen;
    for (int i = 0; i < n_needed; i++) {
        const uint32_t e = needed[i];
        CW_REQUIRE(e < (uint32_t)b->src.n_experts, "bank ensure: expert %u of %d", e, b->src.n_experts);
        if (seen.insert(e).second) want.push_back(e);
    }
    if ((int)want.size() > b->n_slots)
        return cw::set_error(CW_EFULL, "bank: %zu experts needed, %d slots", want.size(), b->n_slots);
    if (int rc = b->refresh()) return rc;
    std::vector<uint8_t> ready((size_t)b->n_slots);
    for (int s = 0; s < b->n_slots; s++) ready[(size_t)s] = b->filling[(size_t)s] ? 0 : 1;
    const size_t n = std::max<size_t>(want.size(), 1);
    std::vector<uint32_t> hits(2 * n), misses(2 * n);
    int nh = 0, nm = 0;
    uint64_t ph = 0;
    const int r = cw_slots_assign(b->slots, want.data(), (int)want.size(), ready.data(), hits.data(), &nh,
                                  misses.data(), &nm, &ph);
    CW_REQUIRE(r >= 0, "bank ensure: bookkeeping refused its arguments");
    if (r == 0) {
        b->st.crowded++;
        return cw::set_error(CW_EFULL, "bank: too few free slots for the %zu experts needed", want.size());
    }
    b->st.hits += (uint64_t)nh;
    b->st.prefetch_hits += ph;
    hipStream_t s = (hipStream_t)stream;
    if (b->fenced && s != b->last) {
        // the table patches a prefetch queued on the previous ensure's stream (its victims taken
        // out) must land before this ensure's own patches, which may list a victim again
        hipError_t w = hipEventRecord(b->handoff, b->last);
        if (w == hipSuccess) w = hipStreamWaitEvent(s, b->handoff, 0);
        if (w != hipSuccess) return cw::set_error(CW_EHIP, "bank: stream wait: %s", hipGetErrorString(w));
    }
    std::vector<uint8_t> waited((size_t)b->n_slots, 0);
    for (int i = 0; i < nh; i++) {
        const uint32_t slot = hits[2 * i + 1];
        if (!b->filling[slot]) continue;
        const hipError_t w = hipStreamWaitEvent(s, b->slot_ev[slot], 0);
        if (w != hipSuccess) return cw::set_error(CW_EHIP, "bank: stream wait: %s", hipGetErrorString(w));
        waited[slot] = 1;
    }
    if (int rc = b->copy_in(misses.data(), nm, s, 0)) {
        // the misses' bytes may not have arrived: they must not count as held
        for (int i = 0; i < nm; i++) cw_slots_release(b->slots, misses[2 * i]);
        return rc;
    }
    b->st.loads += (uint64_t)nm;
    b->st.bytes_loaded += (uint64_t)nm * (uint64_t)b->expert_bytes();
    if (int rc = b->publish(waited, s)) return rc;
    std::fill(b->kept.begin(), b->kept.end(), 0);
    for (int i = 0; i < nh; i++) b->kept[hits[2 * i + 1]] = 1;
    for (int i = 0; i < nm; i++) b->kept[misses[2 * i + 1]] = 1;
    b->last = s;
    b->fenced = true;
    if (n_loaded) *n_loaded = nm;
    return CW_OK;
}

int cw_bank_prefetch(cw_bank *b, const uint32_t *predicted, int n_predicted) {
    CW_REQUIRE(b && n_predicted >= 0 && (n_predicted == 0 || predicted), "bank prefetch: bad arguments");
    if (int rc = b->on_device()) return -rc;
    for (int i = 0; i < n_predicted; i++)
        if (predicted[i] >= (uint32_t)b->src.n_experts)
            return -cw::set_error(CW_EINVAL, "bank prefetch: expert %u of %d", predicted[i], b->src.n_experts);
    if (n_predicted == 0) return 0;
    if (int rc = b->refresh()) return -rc;
    std::vector<uint8_t> ready((size_t)b->n_slots);
    for (int s = 0; s < b->n_slots; s++) ready[(size_t)s] = !b->filling[(size_t)s] && !b->kept[(size_t)s];
    std::vector<uint32_t> out(2 * (size_t)n_predicted);
    const int n = cw_slots_reserve(b->slots, predicted, n_predicted, ready.data(), out.data());
    if (n == 0) return 0;
    if (b->fenced) {
        // everything queued on the ensure stream so far may read the victims' slots: the copies
        // wait for it, and what is queued there later finds the victims absent from the table
        hipError_t w = hipEventRecord(b->fence, b->last);
        if (w == hipSuccess) w = hipStreamWaitEvent(b->copy, b->fence, 0);
        if (w != hipSuccess) {
            for (int i = 0; i < n; i++) cw_slots_release(b->slots, out[2 * i]);
            return -cw::set_error(CW_EHIP, "bank: stream wait: %s", hipGetErrorString(w));
        }
        std::vector<uint8_t> taken((size_t)b->n_slots, 0);
        for (int i = 0; i < n; i++) taken[out[2 * i + 1]] = 1;
        cw::TablePatch p{};
        for (int e = 0; e < b->src.n_experts; e++) {
            const uint32_t v = b->dev_table[(size_t)e];
            if (v == CW_NO_SLOT || !taken[v]) continue;
            b->dev_table[(size_t)e] = CW_NO_SLOT;
            p.expert[p.n] = (uint32_t)e;
            p.slot[p.n] = CW_NO_SLOT;
            if (++p.n == cw::PATCH) {
                hipLaunchKernelGGL(cw::k_table_patch, dim3(1), dim3(64), 0, b->last, b->table, p);
                p.n = 0;
            }
        }
        if (p.n) hipLaunchKernelGGL(cw::k_table_patch, dim3(1), dim3(64), 0, b->last, b->table, p);
        if (int rc = cw::check_launch("k_table_patch")) {
            for (int i = 0; i < n; i++) cw_slots_release(b->slots, out[2 * i]);
            return -rc;
        }
    }
    if (int rc = b->copy_in(out.data(), n, b->copy, 1)) {
        for (int i = 0; i < n; i++) cw_slots_release(b->slots, out[2 * i]);
        return -rc;
    }
    for (int i = 0; i < n; i++) {  // one copy for them all: each slot's event marks its end
        const uint32_t slot = out[2 * i + 1];
        const hipError_t r = hipEventRecord(b->slot_ev[slot], b->copy);
        if (r != hipSuccess) return -cw::set_error(CW_EHIP, "bank: event record: %s", hipGetErrorString(r));
        b->filling[slot] = 1;
    }
    b->st.prefetch_copies += (uint64_t)n;
    return n;
}

int cw_bank_fill_desc(const cw_bank *b, cw_moe_desc *d) {
    CW_REQUIRE(b && d, "bank: null argument");
    for (int m = 0; m < 3; m++) {
        d->dtype[m] = b->src.shrink[m] ? CW_Q2_K : b->src.dtype[m];
        d->w[m] = b->mat[m];
        d->slot_stride[m] = b->slot_eb[m];
    }
    d->slot_table = b->table;
    d->n_slots = b->n_slots;
    return CW_OK;
}

const uint32_t *cw_bank_table(const cw_bank *b) { return b ? b->table : nullptr; }

int cw_bank_slot_of(const cw_bank *b, uint32_t expert) { return b ? cw_slots_slot_of(b->slots, expert) : -1; }

void cw_bank_get_stats(const cw_bank *b, cw_bank_stats *out) {
    if (b && out) *out = b->st;
}

}  // extern "C"
