"""Seeded synthetic inputs for the tests and bench.py: GGUF blocks,
activations and whole models (synth), and a GGUF file writer
(gguf_writer). Not part of the library."""
