"""The IQ tables of include/strata_iq_tables.h as Python lists (parsed at import from the committed header)."""
import os
import re

_SRC = open(os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "include", "strata_iq_tables.h")).read()


def _arr(name):
    m = re.search(r"STRATA_%s\[\d+\] = \{(.*?)\};" % name, _SRC, re.S)
    vals = [v.strip() for v in m.group(1).split(",") if v.strip()]
    return [int(v.rstrip("ul"), 16) if v.startswith("0x") else int(v) for v in vals]


IQ2XXS_GRID = _arr("IQ2XXS_GRID")
IQ3S_GRID = _arr("IQ3S_GRID")
KSIGNS = _arr("KSIGNS_IQ2XS")
KVALUES_IQ4NL = _arr("KVALUES_IQ4NL")
