"""Sampling primitives of the verify path on the GPU (reference: specdec/)."""
