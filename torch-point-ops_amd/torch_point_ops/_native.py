"""Locations of the native libraries of this package."""
import os

_HERE = os.path.dirname(os.path.abspath(__file__))
HIP_LIB = os.path.join(_HERE, "libtpo_hip.so")
TORCH_SHIM = os.path.join(_HERE, "_C.so")
