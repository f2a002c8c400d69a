"""qwen3_5 family on MI355X: config, device cache, model, MTP head, speculative decoder.

Registration mirrors src/qwen3_5/__init__.py:20-23 (model types and sampling defaults).
"""

from .config import Qwen3_5Config, build_config  # noqa: F401
from .kv import Qwen3_5Cache  # noqa: F401
from .modeling_qwen3_5 import Qwen3_5Model  # noqa: F401
from .mtp import MTP, SpecDecoder, generate_mtp, load_mtp, speculate  # noqa: F401
from .weights import load, to_raw  # noqa: F401
from .checkpoint import load_checkpoint, read_checkpoint  # noqa: F401

MODEL_TYPES = ["qwen3_5"]
DEFAULTS = {"temperature": 0.7, "top_p": 0.8, "top_k": 20, "repetition_penalty": 1.05}
