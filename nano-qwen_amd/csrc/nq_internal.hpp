// Host-side helpers shared by the C-ABI entry points: error text, dtype
// codes and argument checks.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/nq_attn.h"

int nq_fail(int code, const char* fmt, ...);
void nq_clear_error();

inline bool nq_dtype_ok(int dt) { return dt == NQ_DTYPE_BF16 || dt == NQ_DTYPE_F32; }
inline int nq_dtype_size(int dt) { return dt == NQ_DTYPE_BF16 ? 2 : 4; }
inline bool nq_aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

// Converts a launch status into the C-ABI return code (negative hipError_t).
int nq_check_launch(hipError_t e);
