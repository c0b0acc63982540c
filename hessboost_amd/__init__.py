"""hessboost-rocm: hessboost's `tree_method=hist` training and batch
prediction on one AMD MI355X (gfx950).

    import hessboost_amd as hb
    model = hb.train({"objective": "binary:logistic", "max_depth": 8, "eta": 0.1},
                     hb.DMatrix(x, label=y), num_boost_round=500)
    p = model.predict(x)
"""
from ._capi import HbrError, lib  # noqa: F401
from .core import (BinnedIndex, Booster, Cuts, DMatrix, DeviceBuffer, Engine, Forest,  # noqa: F401
                   Trainer, train)

__all__ = ["BinnedIndex", "Booster", "Cuts", "DMatrix", "DeviceBuffer", "Engine", "Forest", "HbrError",
           "Trainer", "train"]
