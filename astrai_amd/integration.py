"""Switching an AstrAI model build to this package's HIP FFN layers at run time.

AstrAI builds each decoder block's FFN with ``FFNFactory.create(config.ffn_type,
**cfg)`` (``astrai/model/components/decoder_block.py:29``) from the registry
declared in ``astrai/model/components/mlp.py:10-28``, whose ``register``
refuses a name that is already taken (``astrai/factory.py:84-91``).
``use_hip_ffn`` therefore replaces the registry entries themselves: a model
built afterwards gets this package's ``DeepSeekMoE`` for ``"moe"`` (and, on
request, its ``MLP`` for ``"mlp"``), with the reference's constructor
signature, child modules and ``state_dict`` keys, so its checkpoints load
unchanged. Models built before the call keep the classes they were built with.
``restore_ffn`` puts the previous entries back.

    from astrai_amd.integration import use_hip_ffn
    use_hip_ffn()                 # before the model is built
    model = AutoModel.from_pretrained(path)   # astrai/model/automodel.py:54

``register_kernels`` makes AstrAI's own kernel discovery
(``astrai/extension/loader.py:14-36``) list this package's kernels, so that
``astrai.extension.loader.is_available("moe_route")`` and ``get_module`` answer
for them and ``import astrai.extension.moe_route`` finds them.
"""

from __future__ import annotations

import sys

from astrai_amd.model.components.mlp import MLP, DeepSeekMoE


def _registry(factory):
    if factory is None:
        from astrai.model.components.mlp import FFNFactory as factory  # the reference's registry
    entries = getattr(factory, "_entries", None)
    if not isinstance(entries, dict):
        raise TypeError(f"{factory!r} has no component registry (_entries)")
    return factory, entries


def use_hip_ffn(factory=None, *, moe: bool = True, mlp: bool = False) -> dict:
    """Register the HIP ``DeepSeekMoE`` as ``"moe"`` (and the HIP ``MLP`` as
    ``"mlp"`` when ``mlp`` is set) in ``factory`` (default: AstrAI's
    ``FFNFactory``). Returns the replaced entries, for ``restore_ffn``."""
    factory, entries = _registry(factory)
    chosen = {name: cls for name, cls, on in (("moe", DeepSeekMoE, moe), ("mlp", MLP, mlp)) if on}
    validate = getattr(factory, "_validate_component", None)
    base = getattr(factory, "_component_base", None)
    for cls in chosen.values():  # the registry's base-type check, as its register() does
        if validate is not None:
            validate(cls)
        elif isinstance(base, type) and not issubclass(cls, base):
            raise TypeError(f"{cls.__name__} must inherit from {base.__name__}")
    previous = {name: entries.get(name) for name in chosen}
    entries.update(chosen)
    return previous


def restore_ffn(previous: dict, factory=None) -> None:
    """Undo ``use_hip_ffn``: put back the entries it returned (names that were
    not registered before are removed)."""
    _, entries = _registry(factory)
    for name, cls in previous.items():
        if cls is None:
            entries.pop(name, None)
        else:
            entries[name] = cls


def register_kernels(ext_loader=None) -> list[str]:
    """Add this package's available kernels (``astrai_amd.extension.loader``)
    to a kernel loader with the reference's interface (default: AstrAI's
    ``astrai.extension.loader``): each name is appended to its
    ``KERNEL_NAMES``, marked in ``_available`` and given its module handle in
    ``_modules`` (the dicts its ``is_available`` / ``get_module`` read; the
    reference fills them once, at import, from ``KERNEL_NAMES``), and the
    handle is importable as ``<loader package>.<name>``, the submodule the
    reference's discovery imports. Unavailable kernels are left out. Returns
    the names registered."""
    from astrai_amd.extension import loader as ours

    if ext_loader is None:
        from astrai.extension import loader as ext_loader  # the reference's discovery
    for attr in ("KERNEL_NAMES", "_available", "_modules"):
        if not hasattr(ext_loader, attr):
            raise TypeError(f"{ext_loader!r} has no {attr}: not a kernel loader with the reference's interface")
    package = ext_loader.__package__ or ext_loader.__name__.rpartition(".")[0]
    names = []
    for name in ours.KERNEL_NAMES:
        if not ours.is_available(name):
            continue
        handle = ours.get_module(name)
        if name not in ext_loader.KERNEL_NAMES:
            ext_loader.KERNEL_NAMES.append(name)
        ext_loader._available[name] = True
        ext_loader._modules[name] = handle
        if package:
            sys.modules[f"{package}.{name}"] = handle
        names.append(name)
    return names
