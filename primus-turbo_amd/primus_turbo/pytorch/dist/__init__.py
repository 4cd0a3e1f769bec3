"""Distributed helpers on the FP8 path (mirrors primus_turbo/pytorch/dist/__init__.py)."""

from .fp8_alltoall import *  # noqa: F401,F403
