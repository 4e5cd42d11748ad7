"""CPU oracle for the per-layer ops: test infrastructure (parity checker and
CPU baseline), never imported by the product package."""
