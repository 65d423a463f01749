"""MI355X-native (gfx950) RCSA hot path of CAST: block scoring, top-k block
selection, int8 Q/K quantiser and block-sparse flash attention behind a C ABI
(``include/rcsa.h``, built as ``cast_amd/_lib/librcsa.so``)."""

__version__ = "0.1.0"

__all__ = ["ops", "pipeline", "kernel", "workloads", "layout", "budget", "selector"]
