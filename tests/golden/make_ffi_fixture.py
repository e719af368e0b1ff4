"""Writes llamd_rocm_ffi.json: every function the reference's llamd-rocm crate
binds through `extern "C"` (crates/llamd-rocm/src/{lib,forward,batch,udot}.rs),
with its Rust parameter and return types. Run here, where /root/reference
exists; the tests read only the JSON.

    python tests/golden/make_ffi_fixture.py
"""
import json
import re
from pathlib import Path

SRC = Path("/root/reference/crates/llamd-rocm/src")
OUT = Path(__file__).resolve().parent / "llamd_rocm_ffi.json"


def main() -> None:
    out = {}
    for name in ["lib.rs", "forward.rs", "batch.rs", "udot.rs"]:
        text = (SRC / name).read_text()
        for block in re.finditer(r'extern\s+"C"\s*\{(.*?)\n\s*\}', text, re.S):
            body = re.sub(r"//[^\n]*", "", block.group(1))
            body = re.sub(r"#\[[^\]]*\]", "", body)
            for fn in re.finditer(r"fn\s+(\w+)\s*\((.*?)\)\s*(->\s*([^;]+))?;", body, re.S):
                params = [p.strip() for p in fn.group(2).split(",") if p.strip()]
                types = [p.split(":", 1)[1].strip() for p in params]
                ret = (fn.group(4) or "()").strip()
                out.setdefault(fn.group(1), {"file": f"crates/llamd-rocm/src/{name}",
                                             "params": types, "ret": ret})
    OUT.write_text(json.dumps(out, indent=1, sort_keys=True) + "\n")
    print(f"{len(out)} functions -> {OUT}")


if __name__ == "__main__":
    main()
