// CPU unit test of the allocator bookkeeping (tl_amd/csrc/block_cache.h): streams and events
// are plain integers, and an event counts as completed when the test says so.
#include <cstdio>
#include <cstdlib>
#include <set>

#include "../tl_amd/csrc/block_cache.h"

using tlhip::BlockCache;
using tlhip::block_size_class;

static int failures = 0;
#define CHECK(c)                                                   \
    do {                                                           \
        if (!(c)) {                                                \
            std::printf("FAILED line %d: %s\n", __LINE__, #c);     \
            failures++;                                            \
        }                                                          \
    } while (0)

int main() {
    // size classes: 256-byte granules to 1 MiB, then powers of two
    CHECK(block_size_class(0) == 256);
    CHECK(block_size_class(1) == 256);
    CHECK(block_size_class(256) == 256);
    CHECK(block_size_class(257) == 512);
    CHECK(block_size_class(1 << 20) == (1 << 20));
    CHECK(block_size_class((1 << 20) + 1) == (2 << 20));
    CHECK(block_size_class((3 << 20) - 7) == (4 << 20));

    typedef long Stream;
    typedef long Event;  // 0 = no event
    std::set<Event> done_events, released;
    auto done = [&](Event e) { return done_events.count(e) > 0; };
    auto release = [&](Event e) { released.insert(e); };
    char mem[8];

    {   // one stream, no events: the freed block is reused at once on its own stream
        BlockCache<Stream, Event> c;
        c.put(&mem[0], 256, 1, 0);
        CHECK(c.bytes() == 256 && c.count() == 1);
        CHECK(c.take(512, 1, done, release) == nullptr);  // other class
        CHECK(c.take(256, 1, done, release) == &mem[0]);
        CHECK(c.count() == 0 && c.bytes() == 0);
    }
    {   // freed on stream 1 without an event: never handed to stream 2
        BlockCache<Stream, Event> c;
        c.put(&mem[0], 256, 1, 0);
        CHECK(c.take(256, 2, done, release) == nullptr);
        CHECK(c.count() == 1);
        // ... until the device has been synchronised
        c.mark_all_idle();
        CHECK(c.take(256, 2, done, release) == &mem[0]);
    }
    {   // freed on stream 1 with event 7: stream 2 waits for the event, stream 1 does not
        BlockCache<Stream, Event> c;
        c.put(&mem[1], 256, 1, 7);
        CHECK(c.take(256, 2, done, release) == nullptr);
        done_events.insert(7);
        CHECK(c.take(256, 2, done, release) == &mem[1]);
        CHECK(released.count(7) == 1);  // the event goes back to the pool
        c.put(&mem[2], 256, 1, 8);
        CHECK(c.take(256, 1, done, release) == &mem[2]);  // same stream: no wait
        CHECK(released.count(8) == 1);
    }
    {   // a same-stream block is preferred over another stream's completed one
        BlockCache<Stream, Event> c;
        done_events.insert(9);
        c.put(&mem[3], 1024, 2, 9);
        c.put(&mem[4], 1024, 1, 10);
        CHECK(c.take(1024, 1, done, release) == &mem[4]);
        CHECK(c.take(1024, 1, done, release) == &mem[3]);
        CHECK(c.take(1024, 1, done, release) == nullptr);
    }
    {   // drain hands back every block and event and empties the cache
        BlockCache<Stream, Event> c;
        c.put(&mem[5], 256, 1, 0);
        c.put(&mem[6], 4 << 20, 3, 11);
        int n = 0;
        long evs = 0;
        c.drain([&](void*, Event e) { n++; evs += e; });
        CHECK(n == 2 && evs == 11 && c.count() == 0 && c.bytes() == 0);
    }
    if (failures == 0) std::printf("block cache: all checks passed\n");
    return failures ? 1 : 0;
}
