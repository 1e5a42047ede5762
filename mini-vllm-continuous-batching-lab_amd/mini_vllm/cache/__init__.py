from .pool import MIN_BLOCKS, KVCachePool, compute_num_gpu_blocks

__all__ = ["MIN_BLOCKS", "KVCachePool", "compute_num_gpu_blocks"]
