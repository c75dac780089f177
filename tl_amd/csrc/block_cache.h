// Bookkeeping of the caching device allocator: which freed block may be handed to which
// request.  Plain C++ with no HIP calls, so the policy is unit-tested on the CPU
// (tests/test_block_cache.py builds tests/block_cache_test.cpp against this header).
//
// A block is freed "on a stream": the stream the caller's last use of it was ordered on.
//  * A request on the same stream may reuse it at once -- the stream runs the new work after
//    the old.
//  * A request on another stream may reuse it only once the event recorded at the free has
//    completed (the caller's `done(event)` says so), or once the block has been marked idle
//    (no work pending anywhere: after a device synchronisation).
// Blocks are grouped by size class: 256-byte granules up to 1 MiB, then powers of two.
#pragma once
#include <stddef.h>

#include <map>
#include <utility>

namespace tlhip {

inline size_t block_size_class(size_t b) {
    if (b == 0) b = 1;
    if (b <= (size_t(1) << 20)) return (b + 255) & ~size_t(255);
    size_t c = size_t(1) << 20;
    while (c < b) c <<= 1;
    return c;
}

template <class Stream, class Event>
class BlockCache {
public:
    struct Block {
        void* p;
        Stream stream;  // the stream it was freed on
        Event event;    // recorded on `stream` at the free (null: none recorded)
        bool idle;      // no pending work on any stream
    };

    // Caches block p of class c, freed on stream s with event ev (may be null).
    void put(void* p, size_t c, Stream s, Event ev) {
        blocks_.emplace(c, Block{p, s, ev, false});
        bytes_ += c;
    }

    // A cached block of class c usable on stream s, or nullptr.  Preference: a block freed on
    // s or idle (no wait at all), then one whose free event has completed (done(ev) true).
    // The taken block's event, if any, is handed to release_event.
    template <class Done, class Release>
    void* take(size_t c, Stream s, Done done, Release release_event) {
        auto range = blocks_.equal_range(c);
        for (auto it = range.first; it != range.second; ++it)
            if (it->second.idle || it->second.stream == s) return pop(it, release_event);
        for (auto it = range.first; it != range.second; ++it)
            if (it->second.event && done(it->second.event)) return pop(it, release_event);
        return nullptr;
    }

    // After a device-wide synchronisation: every cached block is free of pending work.
    void mark_all_idle() {
        for (auto& kv : blocks_) kv.second.idle = true;
    }

    // Hands every cached block (and its event) to f(p, event) and empties the cache; only
    // valid when no work that used the blocks is pending.
    template <class F>
    void drain(F f) {
        for (auto& kv : blocks_) f(kv.second.p, kv.second.event);
        blocks_.clear();
        bytes_ = 0;
    }

    size_t bytes() const { return bytes_; }
    size_t count() const { return blocks_.size(); }

private:
    template <class Release>
    void* pop(typename std::multimap<size_t, Block>::iterator it, Release release_event) {
        void* p = it->second.p;
        if (it->second.event) release_event(it->second.event);
        bytes_ -= it->first;
        blocks_.erase(it);
        return p;
    }

    std::multimap<size_t, Block> blocks_;
    size_t bytes_ = 0;
};

}  // namespace tlhip
