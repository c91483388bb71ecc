// protocol.hpp -- the scheduler protocol of the persistent kernels, written
// once for two executors: the gfx950 kernels (through DevPlat in
// pipeline.hpp) and the CPU protocol simulator (apk_amd/sim/, through
// std::atomic-style host primitives, one std::thread per block). It holds
// only the parts whose correctness is a matter of ordering between blocks:
//   - the XCD-aware work queue (exactly-once task hand-out with stealing);
//   - the resume ring of the retreat arm (bounded MPMC ring with per-entry
//     sequence numbers);
//   - which generation a block acts on, and which blocks retreat at it.
// The tile arithmetic, LDS rings and checkpoints stay in the kernels.
//
// The includer defines APK_PROTO_FN (the function qualifiers: device
// inline for the kernels, plain inline for the simulator) and passes a
// platform P with static members:
//   unsigned fetch_add(unsigned*, unsigned)   relaxed, device-wide
//   unsigned load(const unsigned*), int load(const int*)   relaxed
//   void store(int*, int)                     relaxed
//   void acquire()                            device-wide acquire fence
//   void publish_fence()                      orders the caller's earlier
//                                             payload stores (written by the
//                                             platform's publishing stores)
//                                             before its next store
//   int64_t ticks()                           constant-rate clock (100 MHz)
//   void pause()                              back off while spinning
#pragma once
#include <stdint.h>

#include "apk.h"

#ifndef APK_PROTO_FN
#error "APK_PROTO_FN must name the function qualifiers before protocol.hpp is included"
#endif

namespace apk {
namespace proto {

// ---------------------------------------------------------------------------
// XCD-aware work queue. The tile grid (tilesM x tilesN) is walked in a
// grouped order G: bands of GM tile rows, column by column inside a band, so
// that consecutive positions form GM x n blocks of the grid. Positions
// [q*T/8, (q+1)*T/8) of G are XCD q's list; pass p of the task space maps
// position i of list q to task p*T + G(i). A worker pops its own XCD's list
// (counter ctr[q]) and, once that is exhausted, the other lists in turn, so
// every task id below num_tasks is handed out exactly once and task u always
// computes tile u % T.
template <class P>
struct TaskQueue {
  static constexpr int GM = 4;
  unsigned* ctr;
  int tilesM, tilesN, T;
  unsigned numTasks, passes;

  APK_PROTO_FN TaskQueue(unsigned* c, int tm, int tn, unsigned n)
      : ctr(c), tilesM(tm), tilesN(tn), T(tm * tn), numTasks(n),
        passes((n + (unsigned)(tm * tn) - 1) / (unsigned)(tm * tn)) {}

  APK_PROTO_FN int grouped(int i) const {
    const int band = i / (GM * tilesN);
    const int left = tilesM - band * GM;
    const int rows = left < GM ? left : GM;
    const int r = i - band * GM * tilesN;
    return (band * GM + r % rows) * tilesN + r / rows;
  }
  APK_PROTO_FN int list_begin(int q) const {
    return (int)(((long long)q * T) / APK_QUEUE_XCDS);
  }
  // One caller per block. Returns the next task id, or 0xffffffff when every
  // list is exhausted.
  APK_PROTO_FN unsigned pop(int home) const {
    for (int k = 0; k < APK_QUEUE_XCDS; ++k) {
      const int q = (home + k) & (APK_QUEUE_XCDS - 1);
      const int b = list_begin(q), n = list_begin(q + 1) - b;
      if (n == 0) continue;
      const unsigned total = (unsigned)n * passes;
      for (;;) {
        const unsigned j = P::fetch_add(&ctr[q], 1u);
        if (j >= total) break;
        const unsigned u =
            (j / (unsigned)n) * (unsigned)T + (unsigned)grouped(b + (int)(j % (unsigned)n));
        if (u < numTasks) return u;
      }
    }
    return 0xffffffffu;
  }
};

// ---------------------------------------------------------------------------
// Resume queue of the retreat arm: a bounded ring of `cap` entries (cap >= 2),
// tickets [head, tail) in ctl[0..1], in ctl[2] the count of reserved tickets
// not yet claimed, and in ctl[3] the count of tickets reserved and not yet
// released (the ring's occupancy). Entry i = {task, stage, seq, kind << 8 |
// domain} with its checkpoint slot i; ticket t uses entry t % cap. `seq`
// orders the entry's rounds (bounded MPMC ring with per-entry sequence
// numbers): seq == t means free for ticket t, t + 1 published by ticket t's
// producer, and the consumer of ticket t sets it to t + cap once it has read
// the checkpoint back. With cap == 1 "published by t" (t + 1) and "free for
// t + 1" (t + cap) would be the same value, hence cap >= 2.
//
// A producer first takes a unit of occupancy, and only then a ticket: when
// the ring already holds `cap` unreleased tickets it declines the retreat
// without taking one (the block keeps its tile and works on), so every ticket
// taken is published and claimed -- a full ring leaves no hole in the ticket
// order. Occupancy also bounds the wait for the ticket's entry: if at most
// `cap` tickets are unreleased once ticket t is taken, then at least
// t + 1 - cap of the tickets below t have been released, so either ticket
// t - cap (the entry's previous user) is released or some later ticket is --
// and claims go in ticket order, so t - cap has then been claimed by a
// resident block that releases it once its producer has published and its
// checkpoint is read back. Every wait in the ring thus ends on other blocks'
// progress; the deadlines below only keep a block that stopped from hanging
// the grid, and a run that hits one reports it as an error.
// The host sets seq = i for every entry and ctl[0..3] = 0 before a job.
constexpr unsigned RQ_NONE = 0xffffffffu;
constexpr unsigned RQ_FULL = 0xfffffffeu;   // declined: the ring holds cap tickets
constexpr unsigned RQ_STUCK = 0x80000000u;  // flag on a ticket whose entry never freed
// Longest wait for an entry: 20 ms at the 100 MHz clock. A producer
// publishes, and a consumer reads back, within microseconds.
constexpr int64_t RQ_WAIT_TICKS = 2000000;

// Takes a unit of occupancy (or declines: RQ_FULL), then the next ticket with
// one fetch-add (no CAS loop: the producers of one generation arrive
// together, and a CAS loop would serialise them round trip by round trip),
// and waits for its entry to be free -- unless the ticket is its entry's
// first (t < cap), which the host's seq = i set free before the job: a ring
// with an entry for every retreat of a job then takes no second round trip
// before the checkpoint. A ticket whose entry is still taken after `wait`
// ticks (a block holding it stopped) is returned with RQ_STUCK set; the
// caller counts an error and keeps its tile, and the claimant of that ticket
// reports it lost.
template <class P>
APK_PROTO_FN unsigned rq_reserve(unsigned* ctl, unsigned cap, const int* entries,
                                 int64_t wait = RQ_WAIT_TICKS) {
  if (P::fetch_add(&ctl[3], 1u) >= cap) {  // as in rq_pop: give back, decline
    P::fetch_add(&ctl[3], ~0u);
    return RQ_FULL;
  }
  const unsigned t = P::fetch_add(&ctl[1], 1u);
  const int* en = entries + (size_t)(t % cap) * 4;
  if (t >= cap && P::load(&en[2]) != (int)t) {
    const int64_t deadline = P::ticks() + wait;
    while (P::load(&en[2]) != (int)t) {
      if (P::ticks() > deadline) return t | RQ_STUCK;
      P::pause();
    }
  }
  P::fetch_add(&ctl[2], 1u);  // one more ticket to claim
  return t;
}
// Claims the oldest reserved ticket, or RQ_NONE if none is waiting. A claim
// takes one from ctl[2] with a fetch-and-add (and gives it back if there was
// none), then its ticket from the head with another: it never fails and
// retries, however many blocks claim at once. (A compare-and-swap loop on the
// head let one claim through per round trip; with a whole XCD at a tile
// boundary, then a whole continuation grid, claiming at once, it kept them
// from their polls for up to 0.5 ms.) ctl[2] dips below zero while claims
// that found none give theirs back, and no claim takes a ticket that was not
// reserved: a decrement succeeds only from 1 or more, which with the
// give-backs still outstanding means more reservations than claims.
template <class P>
APK_PROTO_FN unsigned rq_pop(unsigned* ctl) {
  if ((int)P::load(&ctl[2]) <= 0) return RQ_NONE;
  if ((int)P::fetch_add(&ctl[2], ~0u) <= 0) {
    P::fetch_add(&ctl[2], 1u);
    return RQ_NONE;
  }
  return P::fetch_add(&ctl[0], 1u);
}
// Once the checkpoint stores of the whole block are complete: the entry's
// fields, the publish fence, then seq = ticket + 1. On gfx950 the slot is
// written through with agent-coherent stores by every thread, each of which
// waits for its stores before the barrier that precedes this call, so the
// fence only orders this thread's field stores before the seq store.
template <class P>
APK_PROTO_FN void rq_publish(int* en, unsigned ticket, int task, int stage, int kind,
                             int domain) {
  P::store(&en[0], task);
  P::store(&en[1], stage);
  P::store(&en[3], (kind << 8) | domain);  // domain: where the retreat freed a CU
  P::publish_fence();
  P::store(&en[2], (int)(ticket + 1));
}
// Waits (bounded) for claimed ticket h to be published; returns its kind + 1,
// or 0 if it was not published within `wait` ticks.
template <class P>
APK_PROTO_FN int rq_wait_ready(const int* en, unsigned h, int64_t wait = RQ_WAIT_TICKS) {
  const int64_t deadline = P::ticks() + wait;
  for (;;) {
    if (P::load(&en[2]) == (int)(h + 1)) {
      P::acquire();
      return (en[3] >> 8) + 1;
    }
    if (P::ticks() > deadline) return 0;
    P::pause();
  }
}
// Once every reader of ticket h's checkpoint is done (their loads complete):
// frees the entry for ticket h + cap, then gives back the ticket's unit of
// occupancy (a producer admitted by it waits for the seq store if it reads
// the entry first).
template <class P>
APK_PROTO_FN void rq_release(unsigned* ctl, int* en, unsigned h, unsigned cap) {
  P::publish_fence();
  P::store(&en[2], (int)(h + cap));
  P::fetch_add(&ctl[3], ~0u);
}

// ---------------------------------------------------------------------------
// Generations. The flag carries a generation number g (event g - 1); a block
// acts on the newest generation it has not seen. A relaunch (continuation)
// joins a running job: generations raised before it started were handled by
// the blocks that saw them, except that a retreat-arm continuation starts
// from the generation it follows (launch_epoch), so that one raised before it
// got its CUs still counts. Returns the block's initial last-seen generation,
// clamped to the event arrays.
APK_PROTO_FN int first_seen(int flag_at_start, int launch_epoch, int num_events) {
  const int seen = launch_epoch > 0 ? launch_epoch : flag_at_start;
  return seen < num_events ? seen : num_events;
}

// Which blocks of the retreat arm retreat at generation f: the first grid,
// by quota, at f = 1 (the first ceil(R / 32) blocks of each domain to start:
// they are chosen as they register, so only they need to poll at every
// site); afterwards only the newest continuation (launched
// after generation launch_epoch, so f > launch_epoch), all of it -- it holds
// the CUs the previous generation freed, and it must complete for the next
// continuation (queued behind it) to start. Every other block keeps working.
enum RetreatRole { RETREAT_NONE = 0, RETREAT_BY_QUOTA = 1, RETREAT_ALL = 2 };
APK_PROTO_FN int retreat_role(bool continuation, int launch_epoch, int f) {
  if (continuation && launch_epoch > 0 && f > launch_epoch) return RETREAT_ALL;
  if (continuation || f != 1) return RETREAT_NONE;
  return RETREAT_BY_QUOTA;
}

}  // namespace proto
}  // namespace apk
