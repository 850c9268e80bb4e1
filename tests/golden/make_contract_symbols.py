"""Writes gpu_contract_symbols.txt: the symbol names the reference's link test
tests/test_gpu_contract.c requires of a non-Apple backend (its table minus the
__APPLE__ branch). Run where /root/reference exists:

    python tests/golden/make_contract_symbols.py
"""
import re
from pathlib import Path

SRC = Path("/root/reference/tests/test_gpu_contract.c")
OUT = Path(__file__).with_name("gpu_contract_symbols.txt")

text = re.sub(r"#ifdef __APPLE__.*?#else", "", SRC.read_text(), flags=re.S)
names = re.findall(r"\(void \(\*\)\(void\)\)(h3_\w+)", text)
OUT.write_text("".join(n + "\n" for n in names))
print(f"{len(names)} symbols -> {OUT}")
