"""MI355X-native batched Hive engine (move generation, FNN features, action
indices, MCTS tree kernels) behind the reference's hive_gpu extension API.

    from hive_neuralnet_amd import hive_gpu
    ext = hive_gpu.load_extension()
"""
from . import hive_gpu  # noqa: F401
from .hive_gpu import load_extension  # noqa: F401

__all__ = ["hive_gpu", "load_extension"]
