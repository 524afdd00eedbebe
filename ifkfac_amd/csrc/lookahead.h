// Helper streams and events of the look-ahead factorisations (linalg.hip's
// fold, gramchol.hip's Gram + Cholesky factor update): one set per device and
// calling stream, created on first use; a factorisation holds the set's lock
// for as long as it enqueues, so two host threads that issue on the same
// calling stream never interleave their event records.
#pragma once
#include <mutex>
#include <vector>

#include "common.h"

namespace ifk {

struct LookAhead {
  std::mutex mu;
  hipStream_t s2 = nullptr;                   // far updates
  hipStream_t s3 = nullptr;                   // bulk work independent of the chain
  std::vector<hipEvent_t> col;                // per-column events (grown on demand)
  hipEvent_t ready[2] = {nullptr, nullptr};   // the block's far operands are written
  hipEvent_t nearwp[2] = {nullptr, nullptr};  // Wp of the next block's columns is formed
  hipEvent_t fall[2] = {nullptr, nullptr};    // all of the block's far update is done
  hipEvent_t done = nullptr;                  // everything queued on s2 so far
  hipEvent_t tready[2] = {nullptr, nullptr};  // T (or M2, N) of the outer block is complete
  hipEvent_t aready[2] = {nullptr, nullptr};  // far part A of the block is applied
};

// The set of the current device and calling stream s (nullptr and *rc set on
// failure).  Sets live until the process ends.
LookAhead* look_ahead(hipStream_t s, int* rc);

// Destroy the set of the current device and calling stream s, after the
// queued work of s and of its helper streams (no set: nothing to do).  Not concurrently with
// a factorisation on s.
int look_ahead_release(hipStream_t s);

// At least n per-column events in la->col (the caller holds la->mu).
int look_ahead_events(LookAhead* la, size_t n);

#define HIPRC(x, what)              \
  do {                              \
    if ((x) != hipSuccess) {        \
      set_error(what);              \
      return IFK_ERR_HIP;           \
    }                               \
  } while (0)

}  // namespace ifk
