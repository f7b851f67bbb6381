// scratch.hpp — the allocation-free MoE step's static device scratch, as seen by the rest of the
// library (host code only).
#pragma once

namespace trc {

// Takes the device address of the scratch array on device `carte` (hipGetSymbolAddress, with that
// device current; the caller's current device is restored) and keeps it for the allocation-free
// step. Once per device; later calls return at once. TRC_OK or the library's error codes.
int preparer_scratch(int carte);

}  // namespace trc
