"""mosship -- Python side of the MI355X MOSS-TTS-Nano LLM decode path and audio codec decoder.

``lib``          ctypes binding of libmoss_hip.so (the C ABI in include/moss_hip.h)
``moss_format``  .moss v1 / state-file formats and the seeded synthetic model
``codec_format`` the codec decoder's tensor list and seeded synthetic decoder
"""
from . import moss_format  # noqa: F401
from .lib import HipBatch, HipCodec, HipLLM, MossHipError, SampleParams, load  # noqa: F401
