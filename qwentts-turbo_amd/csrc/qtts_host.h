// Host-side services shared by the library's persistent kernels (defined in qtts_decode.hip).
#pragma once
#include <hip/hip_runtime.h>
#include <cstddef>
#include <cstdint>

namespace qtts_host {

constexpr uint32_t kSpinCap = 1u << 22;   // ~4 s of polling before an in-kernel wait is declared failed
// Cap of the waits of a launch's first layer pass (~30 ms of polling). Those waits complete only
// once every workgroup has started (the pass's exchanges reach all 32 workgroups of each XCD and
// the 8 XCDs), so they double as an arrival check: a launch that does not find all 256 CUs free
// (kernels of another stream or process holding some) sets the error word within milliseconds,
// every wait that follows gives up at its next check, and every workgroup runs to its end.
constexpr uint32_t kEntrySpinCap = 1u << 15;

// The cap of the first layer pass's waits for the next launch (kEntrySpinCap unless a test set
// another through qtts_debug_entry_spin_cap).
uint32_t entry_spin_cap();

// The current device's set-up check (gfx950, 256 CUs, the workgroup-to-XCD placement), plus room
// for one workgroup of `fn` with `threads` threads on every CU. Cached per device and kernel.
hipError_t check_kernel(const void* fn, int threads, int* device);

// Launch of a persistent kernel (256 workgroups of `threads`) with the single by-value argument
// block `kargs` on `stream`, ordered after the library's previous launch on the device. Before
// the launch, *tag_base receives the tag base of the n_ws workspaces of ws_bytes each at ws
// (zero-filled by a fill kernel on the stream the first time they are used).
hipError_t launch_persistent(const void* fn, int threads, void* kargs, uint32_t* tag_base, void* ws, int n_ws,
                             size_t ws_bytes, hipStream_t stream);

}  // namespace qtts_host
