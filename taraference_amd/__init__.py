"""MI355X (gfx950) batch-1 decode hot path of taraference: HIP kernels behind a
C ABI (include/taraference_hip.h), built in-tree as libtaraference_hip.so."""

__version__ = "0.1.0"
