"""MI355X-native (gfx950) engine for the qwen4_exp token loop.

The engine, kernels and decode runner live in the native library
libcherenkov.so (HIP/C++, C ABI in include/cherenkov/); this package holds
its build script, ctypes bindings and model presets.
"""

from .abi import ChkConfig, ChkOptions, EngineError, lib  # noqa: F401
