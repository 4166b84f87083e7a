// hip_backend.hpp -- the reference-side half of the drop-in: an adi::Backend
// table (include/adi/backend.hpp:10-23) whose entries run on one MI355X through
// the C ABI of include/adi_hip.h.
//
// The table has the signatures of cpu_backend() (src/backend.cpp:11-26), so an
// executor call such as moe_forward(..., hip_backend()) needs no other change
// (docs/architecture.md:52-62). This file is compiled with the reference's own
// headers and linked with libadi_hip.so; it is the only code a maintainer adds.
#pragma once

#include "adi/backend.hpp"

namespace adi {

// The HIP table. Its name is "hip:<cpu order>": the router and head dots follow
// the reduction order of cpu_backend() on this host, so logits and routes are
// bit-identical with it. The first call creates the device context (device
// ADI_HIP_DEVICE, default 0); a missing or non-gfx950 device throws
// std::runtime_error rather than falling back to the CPU.
[[nodiscard]] const Backend &hip_backend();

// Frees every device copy of weights the table has made. The table caches
// copies by host address (the reference's ExpertScratch caches its derived
// tables by source pointer, src/kernels.cpp:33-94), so a caller that unmaps a
// model calls this before mapping another. No counterpart in the reference,
// whose weights are used in place.
void hip_backend_release_weights();

}  // namespace adi
