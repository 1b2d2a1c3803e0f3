from .kda import (
    kda_prepared_varlen_chunk,
    kda_prepared_varlen_recurrent,
    kda_varlen_chunk,
    kda_varlen_chunk_v2,
    kda_varlen_chunk_with_state,
    kda_varlen_recurrent,
    kda_varlen_recurrent_v2,
    prepared_recurrent,
)

__all__ = [
    "kda_prepared_varlen_chunk",
    "kda_prepared_varlen_recurrent",
    "kda_varlen_chunk",
    "kda_varlen_chunk_v2",
    "kda_varlen_chunk_with_state",
    "kda_varlen_recurrent",
    "kda_varlen_recurrent_v2",
    "prepared_recurrent",
]
