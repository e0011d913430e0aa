"""grilly_core — the tape-autograd module (the reference's cpp/python/bindings.cpp surface);
the compiled part is the pybind11 extension _grilly_core built from csrc/bindings.cpp.

torch is imported first when it is installed.  Its HIP libraries ask for the runtime as
`libamdhip64.so` and find the copy it ships; this extension asks for `libamdhip64.so.7`
(ROCm's).  Both carry the soname libamdhip64.so.7: loaded after torch, the extension reuses
torch's runtime; loaded first, it would bring in ROCm's, torch would then load its own, and
two HIP runtimes in one process do not share the device (the second one's calls fail with
"no ROCm-capable device").
"""
try:
    import torch  # noqa: F401
except ImportError:  # C-ABI use without torch: ROCm's runtime serves alone
    pass

import _grilly_core

globals().update({k: getattr(_grilly_core, k) for k in dir(_grilly_core) if not k.startswith("__")})
