"""kokoro_hip: Python front end of the gfx950 decoder + iSTFTNet generator library.

The compute lives in libkokoro_hip.so (HIP kernels + C++ host behind include/kokoro_hip.h);
`api` marshals numpy arrays into that C ABI, `model_spec` and `workloads` build the seeded
random-init weights and synthetic inputs the tests and the benchmark use.
"""
from . import api, model_spec, workloads  # noqa: F401
