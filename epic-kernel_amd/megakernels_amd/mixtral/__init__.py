"""Mixtral batch-1 decode: instruction set, scheduler, launcher, synthetic
weights."""
