"""deltanet_tpu_amd: MI355X-native (gfx950 HIP) drop-in for the forward
delta-rule recurrence core of maelie-labs/deltanet-tpu (chunk_gdn2,
gdn2_decode_step and their variants).  See ``gdn2.py`` for the API."""

from .gdn2 import chunk_gdn2, gdn2_decode_step, gdn2_decode_steps
from .variants import (
    chunk_delta_rule,
    chunk_gdn,
    chunk_gla,
    chunk_kda,
    delta_rule_decode_step,
    gdn_decode_step,
    gla_decode_step,
    kda_decode_step,
)

__version__ = "0.3.0+mi355x.1"

__all__ = [
    "chunk_gdn2",
    "gdn2_decode_step",
    "gdn2_decode_steps",
    "chunk_gdn",
    "gdn_decode_step",
    "chunk_kda",
    "kda_decode_step",
    "chunk_gla",
    "gla_decode_step",
    "chunk_delta_rule",
    "delta_rule_decode_step",
    "__version__",
]
