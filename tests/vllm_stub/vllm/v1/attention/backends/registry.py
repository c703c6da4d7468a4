import enum

REGISTRY = {}


class AttentionBackendEnum(enum.Enum):
    FLASH_ATTN = "FLASH_ATTN"
    TRITON_ATTN = "TRITON_ATTN"
    ROCM_ATTN = "ROCM_ATTN"
    CUSTOM = "CUSTOM"


def register_backend(backend, class_path):
    REGISTRY[backend] = class_path
