from primus_turbo.pytorch.ops.moe.moe_permute import moe_permute, moe_unpermute  # noqa: F401

__all__ = ["moe_permute", "moe_unpermute"]
