import logging


def init_logger(name):
    return logging.getLogger(name)
