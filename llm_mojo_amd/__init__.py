"""llm_mojo_amd: llm_mojo's quantized-weight matmul path on the MI355X.

HIP kernels for gfx950 behind a C ABI (include/llmq.h, libllmq.so), with a
host-side mirror of llm_mojo's format traits (WeightMatrix, KVCache) and its
GPT-2 caller.  There is no CPU fallback: the compute API raises if
libllmq.so is not built.
"""
from ._lib import GGML, LLMQ_BIAS, LLMQ_GELU, LLMQ_RESID, Context, LlmqError, lib  # noqa: F401
from .formats import GGUFFile, act_bytes, act_prepare, linear_act, HipGGUFMatrix, HipQuantMatrix, IntAttnKV, QuantKV8, debug_chunk_sums, debug_read, debug_refmath, head, layernorm, linear, quantize_rows  # noqa: F401
from .gpt2 import GPT2  # noqa: F401
from .llama import TINYLLAMA, Llama  # noqa: F401
