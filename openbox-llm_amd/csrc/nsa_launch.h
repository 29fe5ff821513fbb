// Host-side helpers shared by the C-ABI entry points: status codes, argument
// checks and launch-error capture.  No allocation and no host synchronisation
// happen here; every launch goes to the caller's stream.
#pragma once

#include <hip/hip_runtime.h>

#include "nsa_hip.h"

#define NSA_CHECK(cond, code) \
  do {                        \
    if (!(cond)) return (code); \
  } while (0)

static inline int nsa_launch_status() {
  hipError_t e = hipGetLastError();
  return e == hipSuccess ? NSA_OK : NSA_ERR_LAUNCH;
}
