"""tensorplay_amd: MI355X (gfx950) backend for TensorPlay's P10 reduction + top-k path."""
__version__ = "0.1.0"
