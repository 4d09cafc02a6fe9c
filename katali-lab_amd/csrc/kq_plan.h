// kq_plan.h — host-side launch decisions that need no device, shared by the
// launchers and by CPU tests (plain C++, no HIP headers).
#pragma once

#include <stdint.h>

namespace kq {

// The one-launch layers (the XCD-sliced layer and its stack) wait between
// their workgroups, so all `grid` of them must be resident at once: one per
// CU on a device of exactly `grid` CUs (the slot-to-XCD mapping), with the
// occupancy API's blocks_per_cu for the kernel's block size and LDS at
// least 1.
inline bool xcd_coresident(int cus, int blocks_per_cu, uint32_t grid) {
    return cus > 0 && (uint32_t)cus == grid && blocks_per_cu >= 1 && (uint64_t)blocks_per_cu * (uint64_t)cus >= grid;
}

// Kernel A on a dense FFN: units of 32 h values (a q8_1 block) put
// ceil(units / cus) on the busiest CU; half units put ceil(2 units / cus)
// halves there. Half units when that is less work on the busiest CU and the
// units pair up by eights (384 units on 256 CUs: 2 against 1.5).
inline bool half_units(uint32_t units, uint32_t cus) {
    if (!cus || units % 8) return false;
    const uint64_t full = (units + cus - 1) / cus, half = (2ull * units + cus - 1) / cus;
    return half < 2 * full;
}

}  // namespace kq
