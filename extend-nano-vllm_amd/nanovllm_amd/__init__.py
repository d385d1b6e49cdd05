"""MI355X-native EAGLE3 speculative-decoding step for extend-nano-vLLM.

Public API mirrors nanovllm/__init__.py:8-38 (lazy exports): ``LLM``,
``SamplingParams``, ``Eagle3Config``, ``Eagle3ForCausalLM``,
``load_eagle3_model``.  The hot path (paged verify attention, KV store and
rollback, aux hidden-state gather, argmax + accept) runs in the HIP library
libnanovllm_amd.so; see ``nanovllm_amd.kernels``.
"""

__all__ = (
    "LLM",
    "SamplingParams",
    "Eagle3Config",
    "Eagle3ForCausalLM",
    "load_eagle3_model",
)


def __getattr__(name: str):
    if name == "LLM":
        from nanovllm_amd.llm import LLM

        return LLM
    if name == "SamplingParams":
        from nanovllm_amd.sampling_params import SamplingParams

        return SamplingParams
    if name in {"Eagle3Config", "Eagle3ForCausalLM", "load_eagle3_model"}:
        from nanovllm_amd import eagle3

        return getattr(eagle3, name)
    raise AttributeError(f"module {__name__!r} has no attribute {name!r}")
