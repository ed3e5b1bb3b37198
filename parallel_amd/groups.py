"""Process-group handling for the single-GPU build.

The reference exchanges routed tokens between expert-parallel ranks with
torch.distributed collectives.  This build runs one rank's share on one GPU:
a group of world size 1 (or ``None``) is the identity exchange, and larger
groups are refused with an explicit error rather than silently mis-routed.
"""

from __future__ import annotations

import torch.distributed as dist


def group_size(group) -> int:
    if group is None or not (dist.is_available() and dist.is_initialized()):
        return 1
    return dist.get_world_size(group)


def require_single_rank(group, what: str) -> None:
    size = group_size(group)
    if size != 1:
        raise NotImplementedError(
            f"{what}: this build runs one expert-parallel rank per GPU without collectives; "
            f"a process group of size {size} is not supported"
        )
