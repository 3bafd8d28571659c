"""MI355X-native warm partial-recompute prefill for Qwen2.5-VL (gfx950 HIP kernels).

Public names follow the nano-vllm package the reference builds on:
LLM, SamplingParams (package root), layers.attention.Attention / store_kvcache,
utils.context, engine.model_runner.ModelRunner.  The kernels behind them are
exported through the C ABI in include/vlc_capi.h.
"""
__all__ = ["LLM", "SamplingParams"]


def __getattr__(name):
    if name == "LLM":
        from .llm import LLM

        return LLM
    if name == "SamplingParams":
        from .sampling_params import SamplingParams

        return SamplingParams
    raise AttributeError(name)
