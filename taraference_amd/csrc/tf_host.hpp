// Host-side helpers shared by the C-ABI entry points.
#pragma once
#include <hip/hip_runtime.h>

// Compute units of the current device (cached per device).
int tf_device_cus();

// Workgroups for a persistent grid: `tasks` wave-tasks spread evenly over at
// most (resident workgroups per CU) * CUs workgroups of `threads` threads,
// so that every wave runs the same number of tasks.
// Workgroup size for a staging GEMV with `tasks` wave tasks: enough waves
// per CU to cover the tasks once (a multiple of 256 threads), at most
// max_threads (the kernel's launch bound).  Small GEMVs still reach every
// CU while large ones get one CU-wide workgroup.
int tf_block_threads(int max_threads, long long tasks);
int tf_persistent_blocks(const void* kernel, int threads, int lds_bytes, int tasks);

// Raises a kernel's dynamic LDS limit on the current device to at least
// `bytes` (once per kernel, device and size; thread-safe).  0 or a HIP error.
int tf_set_lds_limit(const void* kernel, int bytes);
