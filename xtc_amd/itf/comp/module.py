# SPDX-License-Identifier: BSD-3-Clause
"""Module interface (src/xtc/itf/comp/module.py:11-106)."""

from __future__ import annotations

from abc import ABC, abstractmethod
from typing import TYPE_CHECKING, Any

if TYPE_CHECKING:
    from ..exec.evaluator import Evaluator
    from ..exec.executor import Executor


class Module(ABC):
    """A compiled, loadable artefact ("shlib" or "executable")."""

    @property
    @abstractmethod
    def file_type(self) -> str: ...

    @property
    @abstractmethod
    def name(self) -> str: ...

    @property
    @abstractmethod
    def payload_name(self) -> str: ...

    @property
    @abstractmethod
    def file_name(self) -> str: ...

    @abstractmethod
    def export(self) -> None: ...

    @abstractmethod
    def get_evaluator(self, **kwargs: Any) -> "Evaluator": ...

    @abstractmethod
    def get_executor(self, **kwargs: Any) -> "Executor": ...
