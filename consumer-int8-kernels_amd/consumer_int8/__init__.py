"""MI355X (gfx950) INT8 linear-layer kernels behind the consumer_int8 operator surface."""

__version__ = "0.1.0"
