"""The encoder's op-by-op oracle composition (lives in oracle/encoder.py, shared with the
CPU baseline of bench.py)."""
from oracle.encoder import (add_layer_norm_ref, attention_ref, dequant_linear, gelu_ref,  # noqa: F401
                            layer_ref)
