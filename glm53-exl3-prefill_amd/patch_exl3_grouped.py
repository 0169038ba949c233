#!/usr/bin/env python3
"""Runtime patch (run before vLLM starts): hook the grouped prefill into vLLM's exl3 overlay module by appending
an env-gated install block to the installed exl3.py; idempotent (kernel/patch_exl3_grouped.py:1-22).

  python patch_exl3_grouped.py [TARGET_EXL3_PY]

TARGET defaults to $EXL3_OVERLAY_PY, else the installed vllm/model_executor/layers/quantization/exl3.py.
The hook imports exl3_grouped_runtime from this file's directory (or $EXL3_GROUPED_DIR) when
EXL3_GROUPED_PREFILL != "0" and calls install() on the overlay module.
"""
import os
import sys
from pathlib import Path

MARKER = "# --- exl3 grouped prefill hook (mi355x) ---"


def hook_block(runtime_dir: str) -> str:
    return f'''

{MARKER}
import os as _gp_os, sys as _gp_sys
if _gp_os.environ.get("EXL3_GROUPED_PREFILL", "0") != "0":
    _gp_dir = _gp_os.environ.get("EXL3_GROUPED_DIR", {runtime_dir!r})
    if _gp_dir not in _gp_sys.path:
        _gp_sys.path.insert(0, _gp_dir)
    import exl3_grouped_runtime as _gp_rt
    _gp_rt.install(_gp_sys.modules[__name__])
'''


def default_target() -> Path:
    env = os.environ.get("EXL3_OVERLAY_PY")
    if env:
        return Path(env)
    import importlib.util
    spec = importlib.util.find_spec("vllm")
    if spec is None or not spec.submodule_search_locations:
        raise SystemExit("vllm is not installed; pass the overlay exl3.py path explicitly")
    return Path(list(spec.submodule_search_locations)[0]) / "model_executor/layers/quantization/exl3.py"


def patch(target: Path, runtime_dir: str | None = None) -> bool:
    """Append the hook to `target` unless present. Returns True if the file was changed."""
    runtime_dir = runtime_dir or os.path.dirname(os.path.abspath(__file__))
    text = target.read_text()
    if MARKER in text:
        print("exl3 grouped prefill hook already present")
        return False
    target.write_text(text + hook_block(runtime_dir))
    print("exl3 grouped prefill hook appended to", target)
    return True


if __name__ == "__main__":
    patch(Path(sys.argv[1]) if len(sys.argv) > 1 else default_target())
