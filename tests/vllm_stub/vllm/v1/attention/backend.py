import enum


class AttentionCGSupport(enum.Enum):
    """How far an attention backend supports full graph capture (vLLM's enum of the same name)."""
    NEVER = 0
    UNIFORM_SINGLE_TOKEN_DECODE = 1
    UNIFORM_BATCH = 2
    ALWAYS = 3
