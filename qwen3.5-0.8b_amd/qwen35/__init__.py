"""Python host of the MI355X Qwen3.5-0.8B decode engine (ctypes over libqwen35.so).

Mirrors the reference's torch-CPU interface (speccheck/specimpl.py:410-517 `Forward`,
speccheck/mtp.py:36-179 `MTPDraft` / `greedy_mtp`) on top of the C ABI in
include/q35.h. There is no CPU fallback: if the HIP library is missing or no GPU is
visible, every entry point raises.
"""
from .engine import (EOS_IDS, VOCAB, Engine, EngineError, Forward, MtpPolicy, State, greedy_mtp,
                     lib_path, load_library, safetensors_scan)

__all__ = ["Engine", "EngineError", "Forward", "MtpPolicy", "State", "greedy_mtp", "load_library",
           "lib_path", "safetensors_scan", "VOCAB", "EOS_IDS"]
