"""Name -> class registry with kwarg-filtered construction.

Keeps the contract of the reference's ``astrai/factory.py:45-147`` that the
MoE layer is created through: ``register(name)`` is a class decorator that
refuses duplicate names and classes outside the factory's declared base type,
and ``create(name, *args, **kwargs)`` drops keyword arguments the component's
``__init__`` does not accept (unless it takes ``**kwargs``), so a caller can
pass a whole model config dict (``decoder_block.py:16-29``).
"""

from __future__ import annotations

import inspect
from typing import Callable, Dict, Generic, List, Type, TypeVar, get_args, get_origin

T = TypeVar("T")


class BaseFactory(Generic[T]):
    """Subclass as ``class MyFactory(BaseFactory[Base]): pass`` to get an
    independent registry whose entries must subclass ``Base``."""

    _entries: Dict[str, type]
    _component_base: type | None = None

    def __init_subclass__(cls, **kwargs):
        super().__init_subclass__(**kwargs)
        for base in getattr(cls, "__orig_bases__", ()):
            if get_origin(base) is BaseFactory:
                (arg,) = get_args(base)
                cls._entries = {}
                cls._component_base = arg if isinstance(arg, type) else None
                return

    @classmethod
    def register(cls, name: str) -> Callable[[Type[T]], Type[T]]:
        def decorator(component_cls: Type[T]) -> Type[T]:
            base = cls._component_base
            if base is not None and not issubclass(component_cls, base):
                raise TypeError(f"{component_cls.__name__} must inherit from {base.__name__}")
            if name in cls._entries:
                raise ValueError(f"Component '{name}' is already registered")
            cls._entries[name] = component_cls
            return component_cls

        return decorator

    @classmethod
    def get_component_class(cls, name: str) -> Type[T]:
        try:
            return cls._entries[name]
        except KeyError:
            raise ValueError(
                f"Unknown component: '{name}'. Supported types: {sorted(cls._entries)}"
            ) from None

    @classmethod
    def create(cls, name: str, *args, **kwargs) -> T:
        component_cls = cls.get_component_class(name)
        params = inspect.signature(component_cls.__init__).parameters.values()
        if not any(p.kind is inspect.Parameter.VAR_KEYWORD for p in params):
            accepted = {p.name for p in params if p.name != "self"}
            kwargs = {k: v for k, v in kwargs.items() if k in accepted}
        return component_cls(*args, **kwargs)

    @classmethod
    def list_registered(cls) -> List[str]:
        return sorted(cls._entries)

    @classmethod
    def is_registered(cls, name: str) -> bool:
        return name in cls._entries
