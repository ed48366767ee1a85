"""Runtime layer: the torch custom ops the engine glue calls (mirror of cuda/src/sglang_exl3/runtime)."""
