"""MI355X-native path-ordered (holonomy) attention forward.

The drop-in module is ``holonomyawareattention_amd.attention_kernel.PathOrderedGeometricMHA``;
it keeps the reference module's constructor and ``forward`` signature and runs
the geometry scan and the attention core as hand-written gfx950 HIP kernels
behind a C ABI (``include/holo_mi355x.h``).
"""
