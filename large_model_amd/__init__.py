"""large_model_amd - MI355X-native Qwen3-MoE expert-FFN layer (libqmsg) for the qms engine.

The compute path is the HIP library ``libqmsg.so`` (gfx950 kernels behind the C ABI declared
in include/qmsg.h). ``large_model_amd.qmsg`` is its Python binding; ``workloads`` holds the
benchmark configurations.
"""
import os

PACKAGE_DIR = os.path.dirname(os.path.abspath(__file__))
REPO_ROOT = os.path.dirname(PACKAGE_DIR)
