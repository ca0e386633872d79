// Host-side helpers shared by the C-ABI entry points: error reporting and
// argument checks.  The error message is thread-local; every entry point
// clears it on entry.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/maxsim_amd.h"

namespace maxsim {

void clear_error();
// Records a printf-style message and returns `code`.
int fail(int code, const char* fmt, ...) __attribute__((format(printf, 2, 3)));
// hipGetLastError() after a launch -> MAXSIM_ERR_LAUNCH with the kernel name.
int check_launch(const char* what);

inline int check_dtype(maxsim_dtype dt) {
  if (dt != MAXSIM_FLOAT32 && dt != MAXSIM_FLOAT16 && dt != MAXSIM_BFLOAT16)
    return fail(MAXSIM_ERR_INVALID, "unknown dtype tag %d", (int)dt);
  return MAXSIM_OK;
}

inline int check_dim(int64_t dim) {
  if (dim <= 0) return fail(MAXSIM_ERR_INVALID, "dim must be > 0; got %lld", (long long)dim);
  if (dim > MAXSIM_AMD_MAX_DIM)
    return fail(MAXSIM_ERR_UNSUPPORTED,
                "dim %lld exceeds the largest supported embedding dim (%d)",
                (long long)dim, MAXSIM_AMD_MAX_DIM);
  return MAXSIM_OK;
}

}  // namespace maxsim
