"""Candidate-slot files for kb_nano's kernel_swapper (tasks/candidate/L1/)."""
