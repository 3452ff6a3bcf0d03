from .transformer import TinyTransformerLM
