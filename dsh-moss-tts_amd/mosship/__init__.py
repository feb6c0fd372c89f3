"""mosship -- Python side of the MI355X MOSS-TTS-Nano LLM decode path.

``lib``          ctypes binding of libmoss_hip.so (the C ABI in include/moss_hip.h)
``moss_format``  .moss v1 / state-file formats and the seeded synthetic model
"""
from . import moss_format  # noqa: F401
from .lib import HipBatch, HipLLM, MossHipError, SampleParams, load  # noqa: F401
