"""ngram_amd: an MI355X-native engine for the n-gram hint path of hermabr/n-gram-hinted-lm.

Host code (Python on PyTorch-ROCm) over a C-ABI HIP library (csrc/, built for gfx950 by ngram_amd.build). Modules:
  data            shard files and the seeded synthetic streams of the benchmark configurations
  lib             the ctypes binding (the reference's Lib convention)
  gpu_val_stats   the validation-side statistics driver (old_records/gpu_val_stats.py on one GPU)
  count_table     corpus-wide exact count tables on the GPU (exact_match CountTable's surface) + hint queries
"""
__all__ = ["data", "lib", "build"]
