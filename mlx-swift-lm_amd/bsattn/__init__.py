"""Block-sparse decode attention for MI355X (gfx950): Python host mirror of the
reference's KVCache / attentionWithCacheUpdate API over libbsattn.so."""
from ._lib import BsattnError, EXPORTS, LIB_PATH, lib
from .attention import attentionWithCacheUpdate
from .cache import BlockSparseKVCache, GenerateParameters, maybeQuantizeKVCache, newCache
from .prompt_cache import loadPromptCache, savePromptCache

__all__ = ["BlockSparseKVCache", "BsattnError", "attentionWithCacheUpdate", "lib", "LIB_PATH",
           "EXPORTS", "savePromptCache", "loadPromptCache", "maybeQuantizeKVCache", "newCache",
           "GenerateParameters"]
