"""MI355X (gfx950) backend for RustLLM's memory-bound tensor ops.

The product is the hipcc-built ``librustllm_hip.so`` behind the C ABI in
``include/rustllm_hip.h``; ``rustllm_amd.abi`` binds it with ctypes.
"""

__all__ = ["abi", "synth"]
