"""Neural-network modules and optimizers."""

from .module import Linear, Module, ReLU, Sequential, Sigmoid, Tanh
from .optimizers import GradientDescent, Optimizer

__all__ = ["GradientDescent", "Linear", "Module", "Optimizer", "ReLU", "Sequential",
           "Sigmoid", "Tanh"]
