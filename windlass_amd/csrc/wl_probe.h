// wl_probe.h - the streaming-read calibration kernel (wl_probe.hip).
#pragma once
#include <hip/hip_runtime.h>

#include <cstdint>

namespace wl {
// Reads bytes / 16 16-byte words of src with `workgroups` workgroups of 256 threads; out (one
// uint32) is written only in a case that does not arise for real data.
hipError_t read_peak_launch(const void *src, int64_t bytes, int workgroups, uint32_t *out, hipStream_t st);
}  // namespace wl
