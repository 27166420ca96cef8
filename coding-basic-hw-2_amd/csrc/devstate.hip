// devstate.hip -- per-device resident state: the CRT constants and the four sticky counters (in
// kCounterSlots slots each) are
// device globals of this code object (each GPU holds its own copy, zero-filled at load), so setting
// a device up needs no device allocation -- one copy of the host-built tables into the global.
#include "common.hpp"

namespace ggemm {
namespace {
__device__ CrtTables g_tables;
__device__ unsigned long long g_counters[kCounterSlots * kCounterStride];
}  // namespace

int device_state(void** tables, void** counters) {
  if (hipGetSymbolAddress(tables, HIP_SYMBOL(g_tables)) != hipSuccess) return 1;
  if (hipGetSymbolAddress(counters, HIP_SYMBOL(g_counters)) != hipSuccess) return 1;
  return 0;
}

}  // namespace ggemm
