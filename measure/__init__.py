"""Measurement tools beside bench.py: the hardware-ceiling probes and the
rocprofv3 summariser. Not part of the libckv product."""
