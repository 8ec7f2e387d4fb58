// The device store of weights derived from the caller's, kept from one call
// to the next: the MI355X form of the reference's store (store.h, store.cc).
//
// A model's weights are the same at every step of a sampler, and deriving a
// form of them -- the quantized bytes, scales, offsets and sums of the bits
// mode's products -- is a pass over all of them at every step; kept, it is
// done once.  The reference keeps its quantized layouts by default, within a
// budget (store.cc:64-99).  Here the caller gives the budget as memory: an
// arena of device memory (sdhip_store_arena), in which the library places its
// entries; with none, nothing is kept and every call derives its form into
// its work buffer, as before.  The library allocates nothing.
//
// An entry is kept for the tensor it was derived from -- its address, type,
// extents and strides -- and for its layout and variant (the bits, the
// groups), as the reference keys them (store.cc:38-57).  It is filled by the
// first call that needs it, on that call's stream, and is ready for every
// later call ordered after it on the device (the same stream, or an event).
// sdhip_forget drops every entry derived from memory that shares a byte with
// the range, as the reference's forget (store.cc:241-266).  No entry is made
// while the stream is being captured into a graph: a graph's replay is not
// the moment the host would mark the entry filled.

#include <hip/hip_runtime.h>

#include <cstring>
#include <map>
#include <mutex>
#include <tuple>

#include "host.h"

namespace sdhip {

namespace {

struct Key {
    const void *begin;
    int32_t type;
    int64_t ne[4];
    int64_t nb[4];
    int32_t layout;
    uint64_t variant;

    auto tie() const {
        return std::tie(begin, type, ne[0], ne[1], ne[2], ne[3], nb[0], nb[1], nb[2], nb[3], layout, variant);
    }
    bool operator<(const Key &o) const { return tie() < o.tie(); }
};

struct Entry {
    size_t offset;  // in the arena
    size_t bytes;
    size_t source;  // the bytes it was derived from
    bool ready;
};

struct State {
    std::mutex mutex;
    char *arena = nullptr;
    size_t size = 0;
    std::map<Key, Entry> entries;
    std::map<size_t, size_t> blocks;  // offset -> bytes, the arena's used parts
    size_t used = 0;
};

State &state() {
    static State *s = new State();  // never destroyed: calls may run to the process's end
    return *s;
}

constexpr size_t kAlign = 256;

// The first gap of the arena that holds `bytes`, or SIZE_MAX.
size_t first_fit(const State &s, size_t bytes) {
    size_t at = 0;
    for (const auto &[offset, n] : s.blocks) {
        if (offset >= at + bytes) return at;
        at = (offset + n + kAlign - 1) / kAlign * kAlign;
    }
    return at + bytes <= s.size ? at : SIZE_MAX;
}

bool overlaps(const void *a, size_t an, const void *b, size_t bn) { return spans_overlap(a, an, b, bn); }

}  // namespace

void *store_entry(const void *begin, int32_t type, const int64_t ne[4], const int64_t nb[4], int32_t layout,
                  uint64_t variant, size_t source, size_t bytes, hipStream_t stream, bool &ready) {
    ready = false;
    State &s = state();
    std::lock_guard<std::mutex> lock(s.mutex);
    if (s.arena == nullptr) return nullptr;
    Key k{};
    k.begin = begin;
    k.type = type;
    std::memcpy(k.ne, ne, sizeof(k.ne));
    std::memcpy(k.nb, nb, sizeof(k.nb));
    k.layout = layout;
    k.variant = variant;
    hipStreamCaptureStatus capture = hipStreamCaptureStatusNone;
    const bool capturing =
        hipStreamIsCapturing(stream, &capture) != hipSuccess || capture != hipStreamCaptureStatusNone;
    const auto it = s.entries.find(k);
    if (it != s.entries.end()) {
        // An entry not yet filled is filled by an eager call only: a captured
        // call would publish it before the graph that fills it has run.
        if (!it->second.ready && capturing) return nullptr;
        ready = it->second.ready;
        return s.arena + it->second.offset;
    }
    if (capturing) return nullptr;
    const size_t at = first_fit(s, bytes);
    if (at == SIZE_MAX) return nullptr;  // past the budget: the call derives into its work buffer
    s.blocks.emplace(at, bytes);
    s.used += bytes;
    s.entries.emplace(k, Entry{at, bytes, source, false});
    return s.arena + at;
}

void store_publish(const void *entry) {
    State &s = state();
    std::lock_guard<std::mutex> lock(s.mutex);
    for (auto &[k, e] : s.entries) {
        if (s.arena + e.offset == entry) e.ready = true;
    }
}

void store_forget(const void *begin, size_t size) {
    State &s = state();
    std::lock_guard<std::mutex> lock(s.mutex);
    if (size == 0) return;
    for (auto it = s.entries.begin(); it != s.entries.end();) {
        if (overlaps(it->first.begin, it->second.source, begin, size)) {
            s.blocks.erase(it->second.offset);
            s.used -= it->second.bytes;
            it = s.entries.erase(it);
        } else {
            ++it;
        }
    }
}

void store_arena(void *arena, size_t bytes) {
    State &s = state();
    std::lock_guard<std::mutex> lock(s.mutex);
    s.entries.clear();
    s.blocks.clear();
    s.used = 0;
    s.arena = bytes > 0 ? static_cast<char *>(arena) : nullptr;
    s.size = s.arena != nullptr ? bytes : 0;
}

size_t store_used(size_t *entries) {
    State &s = state();
    std::lock_guard<std::mutex> lock(s.mutex);
    if (entries != nullptr) *entries = s.entries.size();
    return s.used;
}

}  // namespace sdhip
