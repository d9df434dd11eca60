"""MI355X-native ragged paged attention for micro-vLLM.

A gfx950 HIP library (``_lib/libmvllm_amd.so``, C ABI in
``include/mvllm_amd.h``) behind the reference's ``AttentionOperator``
interface, registered as ``"mi355x_paged"``.
"""

__version__ = "0.1.0"
