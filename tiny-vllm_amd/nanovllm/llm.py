from nanovllm.engine.llm_engine import LLMEngine


class LLM(LLMEngine):
    """User-facing engine (reference: nanovllm/llm.py)."""
