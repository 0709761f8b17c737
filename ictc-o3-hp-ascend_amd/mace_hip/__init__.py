"""MACE-style energy + force model on the ictc_o3 HIP operators (caller side)."""
from .model import MaceICTC
from .runtime import (CapturedEnergyAndForces, CapturedTrainingStep, check_model, configure_model, create_model,
                      energy_and_forces, force_loss, training_step)
from .neighbors import pbc_image_nmax, radius_graph_pbc_gpu
from .structures import radius_graph, sequential_insertion, uniform_box

__all__ = ["MaceICTC", "CapturedEnergyAndForces", "CapturedTrainingStep", "check_model", "configure_model",
           "create_model", "energy_and_forces",
           "force_loss", "training_step", "pbc_image_nmax", "radius_graph", "radius_graph_pbc_gpu",
           "sequential_insertion", "uniform_box"]
