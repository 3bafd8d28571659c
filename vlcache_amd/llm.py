"""LLM entry point (llm.py of the reference: LLM = LLMEngine)."""
from .engine.llm_engine import LLMEngine


class LLM(LLMEngine):
    pass
