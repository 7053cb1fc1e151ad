"""gpt-oss model pieces on MI355X: the MXFP4 MoE block and its configuration.

The reference's model/__init__.py exports GPTOssConfig and GPTOssForCausalLM;
only the MoE block's part of the model exists here.
"""
from .config import GPTOssConfig

__all__ = ["GPTOssConfig"]
