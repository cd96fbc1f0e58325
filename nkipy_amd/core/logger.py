"""Package logger (reference: nkipy/src/nkipy/core/logger.py:6-21), WARNING by default."""

import logging
import os

_LOGGER_NAME = "nkipy"


def get_logger() -> logging.Logger:
    logger = logging.getLogger(_LOGGER_NAME)
    if not logger.handlers:
        h = logging.StreamHandler()
        h.setFormatter(logging.Formatter("[%(name)s] %(levelname)s: %(message)s"))
        logger.addHandler(h)
        logger.setLevel(os.environ.get("NKIPY_LOG_LEVEL", "WARNING").upper())
    return logger
