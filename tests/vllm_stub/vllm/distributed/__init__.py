"""Tensor-parallel rank of the calling worker; tests set TP_RANK / TP_SIZE."""
TP_RANK = 0
TP_SIZE = 1


def get_tensor_model_parallel_rank():
    return TP_RANK


def get_tensor_model_parallel_world_size():
    return TP_SIZE
