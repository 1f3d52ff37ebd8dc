"""MI355X execution backend for KTIR (drop-in for the reference's ``ktir_cpu``
package: ``from ktir_cpu_amd import KTIRInterpreter, HardwareConfig``)."""

from .interpreter import KTIRInterpreter
from .latency import ExecutionModel, HardwareConfig, LatencyCategory, LatencyReport

__all__ = ["KTIRInterpreter", "HardwareConfig", "LatencyReport", "ExecutionModel", "LatencyCategory"]
