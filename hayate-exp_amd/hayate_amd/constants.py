"""Engine constants kept from the reference (hayate/engine/constants.py:8-24)."""

# Accepted compile modes (constants.py:5): on this path compile=True means
# decode ticks replayed from captured HIP graphs, except in the last mode.
COMPILE_MODES = ("default", "reduce-overhead", "max-autotune", "max-autotune-no-cudagraphs")

# Requests admitted into one batch by the reference scheduler (constants.py:8).
MAX_BATCH_SIZE = 20

# Prompt tokens processed per request per tick (constants.py:14).
DEFAULT_PREFILL_CHUNK_SIZE = 512

# Token positions held by the default shared pool (constants.py:17).
DEFAULT_KV_CACHE_TOKENS = 16_384

# Tokens per KV page (constants.py:20).
DEFAULT_KV_PAGE_SIZE = 128

# Smallest page accepted by begin_batch (constants.py:24). The HIP kernels only
# need a multiple of 32; the bound is kept so callers see the same interface.
MIN_KV_PAGE_SIZE = 128

# Qwen3-4B attention geometry (hayate/model/qwen.py:15-31).
NUM_Q_HEADS = 32
NUM_KV_HEADS = 8
HEAD_DIM = 128
RMS_NORM_EPS = 1e-6
ROPE_THETA = 1_000_000
MAX_POSITION_EMBEDDINGS = 40_960
