/*
 * lsamp_testing.h — test hooks of liblsamp.so.  Not part of the production
 * ABI: no reference counterpart, and a production caller must never call
 * anything declared here (the Swift module map does not export this header).
 */
#ifndef LSAMP_TESTING_H
#define LSAMP_TESTING_H

#include "lsamp.h"

#ifdef __cplusplus
extern "C" {
#endif

/* The bounded waits (the fused arrangement's and the top-k kernel's
 * finalizer), process-wide on `device`: polls > 0 makes every wait's target
 * unreachable and gives it up after `polls` polls, so the fail-closed path
 * (LSAMP_ROW_TIMEOUT, token -1) runs while every kernel exits normally;
 * 0 restores normal waits.  While it is set, every fused or top-k row on the
 * device fails closed.  Synchronous; not for use while other calls are in
 * flight. */
lsamp_status lsamp_test_set_spin_limit(int32_t device, int32_t polls);

#ifdef __cplusplus
}
#endif

#endif /* LSAMP_TESTING_H */
