"""MI355X (gfx950) EXL3 routed-expert path of GLM-5.3 behind a C ABI (include/ea_exl3.h).

Modules mirror the reference's Zig launchers: experts (experts.zig), moe (moe.zig), prompt_experts
(prompt_experts.zig), exl3 / linear (exl3.zig, linear.zig), ops (router top-8, SwiGLU). synth makes seeded data.
"""
from ._lib import EaError, LIB_PATH, lib, strerror  # noqa: F401
