"""mdnav — MI355X-native drop-in for the metal-drone-nav RL hot path.

Host-side Python face of the C ABI in include/mdnav.h: ``Sim`` and
``PPOTrainer`` mirror the reference's host classes (main.mm:516-603,
1110-1474) and ``Trainer`` mirrors cpu_reference::Trainer
(cpu_reference.hpp:112-615), all running on the HIP library
``lib/libmdnav.so``.  ``abi`` holds the struct layouts, ``ops`` the stateless
operators.  Importing is cheap; the library loads on first use and raises if
it is missing.
"""
from . import abi  # noqa: F401
from .native import MdnError  # noqa: F401
from .sim import LargePPOTrainer, PPOTrainer, Sim, Trainer, crazyflie_params, load_raptor  # noqa: F401
from . import formats  # noqa: F401
from .evaluate import (bank_evaluate, evaluate_threat, load_bank, sim_evaluate, task_evaluate, task_runtime,  # noqa: F401
                       task_settings)

__all__ = ["abi", "formats", "MdnError", "Sim", "PPOTrainer", "Trainer", "crazyflie_params", "load_raptor",
           "sim_evaluate", "evaluate_threat", "task_evaluate", "task_runtime", "task_settings", "load_bank", "bank_evaluate"]
