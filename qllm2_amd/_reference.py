"""Reference functions install() keeps for calls on CPU tensors.

The HIP library has no CPU path.  The reference's v11 functions compute on
CPU through their own torch code (v11/triton_kernels.py:546-573 picks its
`_pt_*` forms for CPU tensors; v11/flash_pam.py and v11/fused_ce.py are
torch code), so after install() a CPU call of one of this package's
drop-ins runs the function it replaced.  Without install(), or for a
function install() found no reference for, a CPU call raises ValueError.
"""

_SAVED = {}


def save(key, fn):
    """Keep `fn` (a reference function, never one of this package's) under `key`."""
    if callable(fn) and not str(getattr(fn, "__module__", "") or "").startswith("qllm2_amd"):
        _SAVED[key] = fn


def saved(key):
    return _SAVED.get(key)


def on_cpu(key, what, *args, **kwargs):
    """Run the saved reference function `key` on CPU tensors, or raise."""
    fn = _SAVED.get(key)
    if fn is None:
        raise ValueError(f"qpam {what}: tensors must be on the GPU (no CPU path in this library; after "
                         "qllm2_amd.pam_layer.install() CPU calls run the reference's own function)")
    return fn(*args, **kwargs)
