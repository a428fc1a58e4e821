// Host bookkeeping of an expert bank: which expert sits in which slot and which slot goes next.
// Semantics of Slots in crates/engine/src/experts.rs:84-286 (assign 227-248, release 251-258,
// pop 261-269, reserve 273-285, victim 226-229): slots are kept in least-recently-used order;
// a miss takes the least recently used slot that is ready (not being filled) and holds no
// expert the same forward needs; a forward whose misses cannot all be placed changes nothing.
#include <algorithm>
#include <deque>
#include <new>
#include <unordered_map>
#include <unordered_set>
#include <vector>

#include "../../include/cwmoe.h"

struct cw_slots {
    std::vector<uint32_t> holder;                 // CW_NO_SLOT = empty
    std::unordered_map<uint32_t, int> slot_of;
    std::deque<int> lru;                          // least recently used first
    std::unordered_set<uint32_t> prefetched;      // brought in by a guess, not yet asked for

    explicit cw_slots(int n) : holder((size_t)n, CW_NO_SLOT) {
        for (int i = 0; i < n; i++) lru.push_back(i);
    }

    static bool contains(const uint32_t *v, int n, uint32_t e) { return std::find(v, v + n, e) != v + n; }

    bool usable(int slot, const uint8_t *ready, const uint32_t *keep, int n_keep) const {
        if (ready && !ready[slot]) return false;
        return holder[(size_t)slot] == CW_NO_SLOT || !contains(keep, n_keep, holder[(size_t)slot]);
    }

    // position in lru of the slot a miss takes, or -1
    int victim(const uint8_t *ready, const uint32_t *keep, int n_keep) const {
        for (size_t i = 0; i < lru.size(); i++)
            if (usable(lru[i], ready, keep, n_keep)) return (int)i;
        return -1;
    }

    int put(int pos, uint32_t e) {
        const int slot = lru[(size_t)pos];
        lru.erase(lru.begin() + pos);
        const uint32_t old = holder[(size_t)slot];
        if (old != CW_NO_SLOT) {
            slot_of.erase(old);
            prefetched.erase(old);
        }
        holder[(size_t)slot] = e;
        slot_of[e] = slot;
        lru.push_back(slot);
        return slot;
    }

    void touch_back(int slot) {
        lru.erase(std::find(lru.begin(), lru.end(), slot));
        lru.push_back(slot);
    }

    void touch_front(int slot) {
        lru.erase(std::find(lru.begin(), lru.end(), slot));
        lru.push_front(slot);
    }
};

extern "C" {

cw_slots *cw_slots_new(int n_slots) {
    if (n_slots <= 0) return nullptr;
    return new (std::nothrow) cw_slots(n_slots);
}

void cw_slots_free(cw_slots *s) { delete s; }

int cw_slots_assign(cw_slots *s, const uint32_t *needed, int n_needed, const uint8_t *ready, uint32_t *hits, int *n_hits,
                    uint32_t *misses, int *n_misses, uint64_t *prefetch_hits) {
    if (!s || n_needed < 0 || (n_needed && !needed) || !hits || !misses || !n_hits || !n_misses) return -1;
    int missing = 0;
    for (int i = 0; i < n_needed; i++) missing += s->slot_of.count(needed[i]) ? 0 : 1;
    int free_slots = 0;
    for (int slot : s->lru) free_slots += s->usable(slot, ready, needed, n_needed) ? 1 : 0;
    if (free_slots < missing) return 0;
    int nh = 0, nm = 0;
    uint64_t ph = 0;
    for (int i = 0; i < n_needed; i++) {
        const uint32_t e = needed[i];
        auto it = s->slot_of.find(e);
        if (it != s->slot_of.end()) {
            s->touch_back(it->second);
            if (s->prefetched.erase(e)) ph++;
            hits[2 * nh] = e;
            hits[2 * nh + 1] = (uint32_t)it->second;
            nh++;
            continue;
        }
        const int pos = s->victim(ready, needed, n_needed);  // exists: free_slots >= missing
        misses[2 * nm] = e;
        misses[2 * nm + 1] = (uint32_t)s->put(pos, e);
        nm++;
    }
    *n_hits = nh;
    *n_misses = nm;
    if (prefetch_hits) *prefetch_hits = ph;
    return 1;
}

void cw_slots_release(cw_slots *s, uint32_t expert) {
    if (!s) return;
    auto it = s->slot_of.find(expert);
    if (it == s->slot_of.end()) return;
    const int slot = it->second;
    s->slot_of.erase(it);
    s->holder[(size_t)slot] = CW_NO_SLOT;
    s->prefetched.erase(expert);
    s->touch_front(slot);
}

void cw_slots_pop(cw_slots *s, const uint32_t *used, int n) {
    if (!s || !used) return;
    for (int i = 0; i < n; i++) {
        auto it = s->slot_of.find(used[i]);
        if (it != s->slot_of.end()) s->touch_front(it->second);
    }
}

int cw_slots_reserve(cw_slots *s, const uint32_t *predicted, int n_predicted, const uint8_t *ready, uint32_t *out) {
    if (!s || n_predicted < 0 || (n_predicted && (!predicted || !out))) return 0;
    int n = 0;
    for (int i = 0; i < n_predicted; i++) {
        const uint32_t e = predicted[i];
        if (s->slot_of.count(e)) continue;
        const int pos = s->victim(ready, predicted, n_predicted);
        if (pos < 0) continue;
        const int slot = s->put(pos, e);
        s->prefetched.insert(e);
        out[2 * n] = e;
        out[2 * n + 1] = (uint32_t)slot;
        n++;
    }
    return n;
}

uint32_t cw_slots_holder(const cw_slots *s, int slot) {
    if (!s || slot < 0 || (size_t)slot >= s->holder.size()) return CW_NO_SLOT;
    return s->holder[(size_t)slot];
}

int cw_slots_slot_of(const cw_slots *s, uint32_t expert) {
    if (!s) return -1;
    auto it = s->slot_of.find(expert);
    return it == s->slot_of.end() ? -1 : it->second;
}

void cw_slots_lru(const cw_slots *s, int *order) {
    if (!s || !order) return;
    int i = 0;
    for (int slot : s->lru) order[i++] = slot;
}

int cw_slots_is_prefetched(const cw_slots *s, uint32_t expert) { return s && s->prefetched.count(expert) ? 1 : 0; }

void cw_slots_table(const cw_slots *s, uint32_t *table, int n_experts) {
    if (!s || !table) return;
    for (int e = 0; e < n_experts; e++) table[e] = CW_NO_SLOT;
    for (const auto &kv : s->slot_of)
        if (kv.first < (uint32_t)n_experts) table[kv.first] = (uint32_t)kv.second;
}

}  // extern "C"
