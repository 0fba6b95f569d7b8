// Helpers shared by the library's host sources (not part of the C ABI).
#pragma once

#include <stdint.h>

#include <vector>

#include "../../include/pwfp8.h"
#include "pw_device.h"

namespace pw {

// Records a printf-style message as the calling thread's last error and returns code.
int fail(int code, const char *fmt, ...);
// Makes the runtime's device current: PW_OK or PW_ERR_DEVICE.
int set_device_of(pw_runtime *rt);
// A bank over `table` (one ExpertPtrs per expert) that owns the device allocation `owned`.
int make_owned_bank(pw_runtime *rt, const std::vector<ExpertPtrs> &table, uint32_t hidden, uint32_t intermediate,
                    void *owned, uint64_t owned_bytes, pw_expert_bank **out);

}  // namespace pw
