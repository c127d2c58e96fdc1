"""Python plumbing around libgemma4_sampler.so (the MI355X sampler for the
Gemma4.pas engine): ctypes bindings for the sampler, the HIP runtime and the
synthetic workload generators.  The product is the C ABI in
include/gemma4_sampler.h; this package only drives it."""
from . import hip, native, workload  # noqa: F401
from .native import (Sampler, TSamplingParams, SamplerError, DeviceOutputs,  # noqa: F401
                     DTYPE_F32, DTYPE_BF16)
