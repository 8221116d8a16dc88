"""AdaLN modulation tables from precomputed schedule files (the reference's x_base/x_base/adaln_cache)."""
from .cache import (MODALITY_NUM, AdalnScheduleCache, BlockTables, adaln_indices, install_adaln_cache)

__all__ = ["AdalnScheduleCache", "BlockTables", "MODALITY_NUM", "adaln_indices", "install_adaln_cache"]
