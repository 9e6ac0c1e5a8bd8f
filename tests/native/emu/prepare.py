"""Turn the gfx950 kernel source into a host C++ translation unit for the wave
emulator (tests only).  Four mechanical rewrites, nothing else:

* dynamic LDS (`extern __shared__ T name[];`) becomes a pointer to the
  emulated workgroup's LDS;
* each static LDS array (`__shared__ T a[N];`) becomes a pointer to a
  per-workgroup emulated object (guarded, poisoned, counted against the
  160 KB a workgroup can hold);
* the empty asm statements that pin values in scalar registers (an AMDGPU
  register constraint) are dropped;
* LDS address-space casts become plain pointer casts;

and the include of the C ABI header is made search-path relative.
"""

from __future__ import annotations

import re
import sys


_STATIC_LDS = re.compile(r"^(\s*)__shared__ (?:__attribute__\(\(aligned\(\d+\)\)\) )?(\w+) ([^;]+);", re.M)


def _static_lds(src: str) -> tuple[str, int]:
    """`__shared__ T a[N], b[M];` -> per-workgroup emulated LDS objects."""
    count = 0

    def one(m: re.Match) -> str:
        nonlocal count
        indent, ty, decls = m.group(1), m.group(2), m.group(3)
        out = []
        for d in re.findall(r"(\w+)\[([^\]]+)\]", decls):
            out.append(f"{ty}* {d[0]} = ({ty}*)emu::static_lds({count}, sizeof({ty}) * ({d[1]}));")
            count += 1
        return indent + " ".join(out)

    return _STATIC_LDS.sub(one, src), count


def transform(src: str) -> str:
    src, n_static = _static_lds(src)
    if n_static == 0:
        raise ValueError("kernel source changed shape: no static LDS objects found")
    out, n_lds = re.subn(r"extern __shared__ (?:__attribute__\(\(aligned\(\d+\)\)\) )?(\w+) (\w+)\[\];",
                         r"\1* \2 = (\1*)emu::dyn_lds();", src)
    out, n_asm = re.subn(r'asm volatile\(""\s*::"s"[^;]*\);', "", out)
    out, n_as = re.subn(r"\(void __attribute__\(\(address_space\(3\)\)\)\*\)", "(void*)", out)
    out, n_inc = re.subn(r'#include "\.\./\.\./include/w4a16\.h"', '#include "w4a16.h"', out)
    if min(n_lds, n_asm, n_as, n_inc) == 0:
        raise ValueError(f"kernel source changed shape: rewrites {n_lds} {n_asm} {n_as} {n_inc}")
    return out


if __name__ == "__main__":
    with open(sys.argv[1]) as f:
        text = transform(f.read())
    with open(sys.argv[2], "w") as f:
        f.write(text)
