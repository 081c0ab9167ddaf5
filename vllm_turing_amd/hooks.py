"""How the package attaches itself to vLLM: replacing an attribute of a vLLM module or class by this package's
function, once, and recording what was replaced.

The reference patches vLLM at plugin load (vllm_turing/__init__.py:38-72), each hook in its module's install() and
each guarded by a marker attribute so a second install() is a no-op (w8a8.py:129-130, quantfuse.py:30-31,
lmhead.py:114-116), and only on the GPU its kernels are built for (sm75 there, w8a8.py:131-133, lmhead.py:108-110).
Here every install() goes through replace(), which marks the new function, keeps the replaced one as `_orig`, refuses
to wrap its own function twice and appends (owner, name) to INSTALLED in the order the hooks went in; on_gfx950() is
the one device gate.
"""
import torch

INSTALLED = []          # (owner name, attribute) of every replacement made, in order
MARK = "_vllm_turing"


def on_gfx950() -> bool:
    """Whether the current device is an MI355X-class gfx950 GPU (the only target the kernels are built for)."""
    if not torch.cuda.is_available():
        return False
    try:
        return "gfx950" in torch.cuda.get_device_properties(torch.cuda.current_device()).gcnArchName
    except (RuntimeError, AttributeError):
        return False


def ours(fn) -> bool:
    return bool(getattr(fn, MARK, False))


def replace(owner, name: str, fn) -> bool:
    """owner.<name> = fn, with fn marked as this package's and fn._orig = the replaced attribute.  Does nothing if
    owner.<name> already is one of this package's functions.  Returns True when the attribute is ours afterwards."""
    cur = getattr(owner, name, None)
    if ours(cur):
        return True
    setattr(fn, MARK, True)
    fn._orig = cur
    setattr(owner, name, fn)
    INSTALLED.append((getattr(owner, "__name__", type(owner).__name__), name))
    return True
