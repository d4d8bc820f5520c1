"""InferenceSession with the HIP backend (the reference's session.py:10-125 and
backends/base.py:12-37).

``InferenceSession(graph, backend="hip")`` compiles the graph to an
``.aexrt`` engine (W8A8 on every int8-eligible conv unless an explicit
``algo_map`` is given) and runs it through libaexrt_hip.so.  ``"auto"``
resolves to ``"hip"``; there is no CPU backend here, so a missing library or
GPU raises instead of silently running elsewhere.
"""
from __future__ import annotations

from abc import ABC, abstractmethod
from dataclasses import dataclass
from typing import Any, Dict, Optional

import numpy as np

from .graph import Graph


@dataclass(frozen=True)
class BackendInfo:
    name: str
    device: str
    capabilities: Dict[str, Any]


class Backend(ABC):
    name = "backend"

    @abstractmethod
    def info(self) -> BackendInfo: ...

    @abstractmethod
    def prepare(self, graph: Graph) -> None: ...

    @abstractmethod
    def run(self, inputs: Dict[str, Any]) -> Dict[str, Any]: ...


class HipBackend(Backend):
    """Runs a graph as one compiled engine on an MI355X."""

    name = "hip"

    def __init__(self, precision: str = "fp16", w8a8: bool = True, algo_map: Optional[Dict[int, int]] = None,
                 int8_convs: Optional[list] = None, device_index: int = 0) -> None:
        self.precision = precision
        self.w8a8 = w8a8
        self.algo_map = algo_map
        self.int8_convs = int8_convs
        self.device_index = device_index
        self.model = None
        self.engine_bytes: Optional[bytes] = None
        self.graph: Optional[Graph] = None

    def info(self) -> BackendInfo:
        caps = self.model.capabilities if self.model is not None else {}
        return BackendInfo(self.name, f"hip:{self.device_index}", caps)

    def prepare(self, graph: Graph) -> None:
        from . import engine as E
        from .runtime import NativeHipYoloModel

        self.graph = graph
        algo = self.algo_map
        if algo is None and self.w8a8:
            replay = E.lower_graph(graph)
            names = self.int8_convs
            if names is None and graph.metadata.get("int8_convs"):
                names = graph.metadata["int8_convs"].split(",")
            algo = E.w8a8_algo_map(replay, names)
        self.engine_bytes = E.build_aexrt_engine(graph, precision=self.precision, algo_overrides=algo)
        self.model = NativeHipYoloModel(self.engine_bytes, self.device_index)

    def run(self, inputs: Dict[str, Any]) -> Dict[str, Any]:
        (name, x), = inputs.items()
        self.model.run(np.asarray(x, dtype=np.float32))
        out = self.model.output()
        spec_shape = self._output_shape()
        return {self.graph.outputs[0]: out.reshape(spec_shape)}

    def _output_shape(self):
        from .graph import infer_value_specs

        return infer_value_specs(self.graph)[self.graph.outputs[0]].shape


class InferenceSession:
    """Compiled inference session (session.py:10-125)."""

    def __init__(self, graph: Graph, backend: str = "auto", device: str = "auto", optimize: bool = True,
                 **backend_kwargs: Any) -> None:
        self.original_graph = graph
        self.graph = graph.clone()
        self.backend_name = "hip" if backend == "auto" else backend
        self.backend = self._make_backend(self.backend_name, device, backend_kwargs)
        self.backend.prepare(self.graph)

    def _make_backend(self, backend: str, device: str, kwargs: Dict[str, Any]) -> Backend:
        if backend in ("hip", "rocm", "mi355x"):
            idx = 0
            if device not in ("auto", "cuda", "hip") and ":" in device:
                idx = int(device.split(":", 1)[1])
            return HipBackend(device_index=idx, **kwargs)
        raise ValueError(f"unknown backend: {backend} (this package provides 'hip')")

    def info(self) -> BackendInfo:
        return self.backend.info()

    def run(self, inputs: Dict[str, Any]) -> Dict[str, Any]:
        missing = set(self.graph.inputs) - set(inputs)
        if missing:
            raise ValueError(f"missing inputs: {sorted(missing)}")
        return self.backend.run(inputs)
