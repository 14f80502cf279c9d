"""Dispatch layer with the reference's public surface (dispatcher/__init__.py:8-11):
``KernelDispatcher`` and ``get_registry``; REST app in ``.api``, CLI in ``.cli``."""
from .dispatcher import KernelDispatcher
from .registry import get_registry

__all__ = ["KernelDispatcher", "get_registry"]
