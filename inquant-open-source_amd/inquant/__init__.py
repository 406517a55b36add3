"""InQuant packed-KV hot path on MI355X (gfx950).

Drop-in host modules for the reference package `inquant`: codec (K4 keys),
value_codec (V2/V4 values), cache (InQuantCache), triton_selection
(reuse_map) and triton_attention (PackedDecodeState).  The kernels live in
libinquant_hip.so beside this file; nothing falls back to CPU code.
"""

__version__ = "0.1.0"
