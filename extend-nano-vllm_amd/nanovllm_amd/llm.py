"""``LLM`` is the engine itself (nanovllm/llm.py:4-5)."""
from nanovllm_amd.engine.llm_engine import LLMEngine


class LLM(LLMEngine):
    pass
