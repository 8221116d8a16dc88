"""Head-parallel attention transport (the reference's x_base/x_base/phaa package): the per-row
FP8 wire codec around the sequence-parallel all-to-all."""
