// Host-side check of the XCD-local split-K ticket arithmetic (q4_common.h):
// for every split count S <= 16 and seeded placements of the splits on the
// eight XCDs, in random arrival orders, the arrival count reaches S exactly at
// the last arrival and the last arrival's local mask holds exactly the splits
// placed on its own XCD.  Prints "ok" and exits 0, or the failing case and 1.
#include <cstdio>
#include <cstdlib>

#include "q4_common.h"

int main() {
    unsigned rng = 12345u;
    auto next = [&]() { rng = rng * 1664525u + 1013904223u; return rng >> 8; };
    for (int S = 1; S <= mcq4::XCD_SPLIT_MAX; ++S) {
        for (int trial = 0; trial < 2000; ++trial) {
            unsigned xcc[16], order[16];
            const int mode = trial % 4;   // 0: all local, 1: one foreign, 2: random, 3: all on XCD 7
            const unsigned home = next() % 8;
            for (int q = 0; q < S; ++q) xcc[q] = mode == 0 ? home : mode == 3 ? 7u : next() % 8;
            if (mode == 1) xcc[next() % S] = (home + 1 + next() % 7) % 8;
            for (int q = 0; q < S; ++q) order[q] = q;
            for (int q = S - 1; q > 0; --q) { int r = next() % (q + 1); unsigned t = order[q]; order[q] = order[r]; order[r] = t; }
            uint64_t ticket = 0;
            for (int a = 0; a < S; ++a) {
                const int sp = order[a];
                const uint64_t inc = mcq4::xcd_ticket_inc(xcc[sp], sp);
                const uint64_t prev = ticket;
                ticket += inc;
                const bool last = (prev & 0xFF) == (uint64_t)(S - 1);
                if (last != (a == S - 1)) { printf("S=%d trial=%d: last flag at arrival %d\n", S, trial, a); return 1; }
                if (!last) continue;
                uint32_t want = 0;
                for (int q = 0; q < S; ++q) if (xcc[q] == xcc[sp]) want |= 1u << q;
                const uint32_t got = mcq4::xcd_ticket_local_mask(ticket, xcc[sp], S);
                if (got != want) { printf("S=%d trial=%d: mask %x want %x\n", S, trial, got, want); return 1; }
            }
        }
    }
    printf("ok\n");
    return 0;
}
