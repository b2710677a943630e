"""MI355X-native VoroTracing traversal hot path.

``vorotracing_amd._C`` is the drop-in for the reference's ``_C`` extension
module; ``vorotracing_amd.ops`` mirrors ``vorotracing.cuda``;
``vorotracing_amd.infer`` holds the inference preparation and render caller
(``VoroTracingInfer``) and ``vorotracing_amd.model`` the training caller
(``VoroTracing.forward``).  The kernels live in ``csrc/`` (HIP, gfx950) and
are reached through the C ABI of ``libvt_hip.so`` (include/vt_abi.h).
"""

__version__ = "0.1.0"
