"""quicklm_amd: MI355X (gfx950) decode engine for QuickLM's hybrid
Gated-DeltaNet / GQA transformer.

Native parts (built in-tree by `python -m quicklm_amd.build`):
  libqlm_hip.so     hand-written HIP kernels behind the C ABI in include/qlm_hip.h
  libqlm_engine.so  C++17 host engine (loader, model, graph-captured decode
                    loop) behind the C ABI in include/qlm_engine.h

`quicklm_amd.hip` and `quicklm_amd.engine` are thin ctypes bindings of those
two ABIs; they raise when the libraries are missing (no CPU fallback).
"""

__all__ = ["hip", "engine", "synth"]
