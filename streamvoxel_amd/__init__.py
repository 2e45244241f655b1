"""MI355X-native StreamVoxel per-step generation hot path.

`streamvoxel_amd.sampling` mirrors `streamvoxel.sampling` (entropy, block quota, low-entropy-last, schedules) and
`streamvoxel_amd.stream` mirrors the hot-path parts of `streamvoxel.stream` (fast_ops: no-sync selection, the
graph-capturable slot, packed cross-attention keys; slot: the low-entropy-last state machine). Device work runs in
libsvhip.so (hand-written gfx950 HIP kernels behind the C ABI in include/svhip.h).
"""
from streamvoxel_amd._lib import load  # noqa: F401

__version__ = '0.1.0'
