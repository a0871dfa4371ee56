"""CPU oracle for the block-FP8 linear path -- test infrastructure only."""
