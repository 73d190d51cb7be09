"""MI355X (gfx950) backend of the lfm3-kv800 800h compressed KV-cache path.

Modules: kv800 (the reference's cache / quantizer / decode API, kv800.py, with the `hip` backend), kv800_hip (ctypes
binding of the C-ABI library libkv800_hip.so built from csrc/ by build.py), vllm_cache (the vLLM attention backend's
per-step cache work on the device: new-token rows, sinks, flush, decode tables, decode and prefill rows of a mixed
batch), train (patch_for_training's fake quantization on the GPU), model / model_ops (an LFM3-shaped engine loop that
drives every attention layer through the above).
Kept free of torch imports, like the reference package (lfm3_kv800/__init__.py:1-6)."""
import logging

__version__ = "0.1.1"


def get_logger() -> logging.Logger:
    """Package logger with its own handler (INFO lines also appear in worker processes), as lfm3_kv800/__init__.py:12-21."""
    lg = logging.getLogger("lfm3_kv800_amd")
    if not lg.handlers:
        h = logging.StreamHandler()
        h.setFormatter(logging.Formatter("%(levelname)s %(asctime)s [lfm3_kv800_amd] %(message)s", "%m-%d %H:%M:%S"))
        lg.addHandler(h)
        lg.setLevel(logging.INFO)
        lg.propagate = False
    return lg
