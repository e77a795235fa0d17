"""MI355X-native MoE feed-forward engine with the ``moe_dispatch`` API.

Forward-only operators on hand-written gfx950 HIP kernels, loaded from the
prebuilt ``libmoe_hip.so`` on first GPU use; importing the package never
compiles or touches the GPU. Public names follow the reference package
(``src/moe_dispatch/__init__.py:6-23``).
"""

from importlib import import_module

__version__ = "0.1.0"
__all__ = ["dispatch", "combine", "PackedTokens", "CudaWorkspace", "TorchWorkspace", "MoEBlock",
           "MoEConfig"]
_EXPORTS = {
    "dispatch": (".ops", "dispatch"),
    "combine": (".ops", "combine"),
    "PackedTokens": (".ops", "PackedTokens"),
    "CudaWorkspace": (".workspace", "CudaWorkspace"),
    "TorchWorkspace": (".reference", "TorchWorkspace"),
    "MoEBlock": (".layer", "MoEBlock"),
    "MoEConfig": (".layer", "MoEConfig"),
}


def __getattr__(name):
    if name not in _EXPORTS:
        raise AttributeError(f"module {__name__!r} has no attribute {name!r}")
    module, symbol = _EXPORTS[name]
    value = getattr(import_module(module, __name__), symbol)
    globals()[name] = value
    return value
