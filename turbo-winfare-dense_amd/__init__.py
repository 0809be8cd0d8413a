"""MI355X (gfx950) token-selection path for Turbo-WinFare Dense.

The directory name is not a Python identifier; load it with
``importlib.import_module("turbo-winfare-dense_amd")`` after putting the repository root on
``sys.path``. Everything lives in the ``twd`` submodule (ctypes over libtwd_head.so).
"""
from .twd import *  # noqa: F401,F403
from .twd import (LMHead, Selector, SamplingParams, SpeculativeCoordinator, RowParams,  # noqa: F401
                  apply_repetition_penalty, sample_token, seed_for, splitmix64,
                  validate_sampling, uniform_from_seed, generate_head, head_bytes, decode_verify,
                  TwdError, G4DenseFormatError, LIB_PATH)
