"""Writes reference_kernel_abi.json: the parameter list of every kernel the
reference instantiates (POPCORN_INSTANTIATE_KERNEL in
Sources/Popcorn/Kernels/**/*.metal), as device-pointer count and the byte
size of each constants block after them (PopcornKernelTypes.h structs: every
field is 4 bytes), with the source line of the kernel template. Reads the
reference's Metal and header sources as text; run from a checkout that has
them (default /root/reference)."""
import glob
import json
import os
import re
import sys

REF = sys.argv[1] if len(sys.argv) > 1 else "/root/reference"
SRC = os.path.join(REF, "Sources")


def struct_sizes(text):
    sizes = {}
    for m in re.finditer(r"typedef struct \{(.*?)\}\s*(\w+);|struct\s+(\w+)\s*\{(.*?)\};", text, re.S):
        body, name = (m.group(1), m.group(2)) if m.group(2) else (m.group(4), m.group(3))
        fields = [f for f in re.sub(r"//[^\n]*", "", body).split(";") if f.strip()]
        sizes[name] = 4 * len(fields)
    return sizes


def main():
    sizes = struct_sizes(open(os.path.join(SRC, "PopcornShaderTypes", "PopcornKernelTypes.h")).read())
    templates, names = {}, {}
    for path in sorted(glob.glob(os.path.join(SRC, "Popcorn", "Kernels", "**", "*.metal"), recursive=True)):
        raw = open(path).read()
        rel = os.path.relpath(path, REF)
        text = re.sub(r"//[^\n]*", "", raw)
        text = re.sub(r"\[\[.*?\]\]", "", text)
        sizes.update({k: v for k, v in struct_sizes(text).items() if k not in sizes})
        for m in re.finditer(r"kernel\s+void\s+(\w+)\s*\((.*?)\)\s*\{", text, re.S):
            params = []
            for p in re.split(r",\s*(?![^<]*>)", m.group(2)):
                p = p.strip()
                if p.startswith("device"):
                    params.append(("ptr", 8))
                elif p.startswith("constant"):
                    params.append(("val", re.search(r"constant\s+(\w+)\s*&", p).group(1)))
            line = raw[: raw.find("kernel void " + m.group(1))].count("\n") + 1
            templates[m.group(1)] = (params, f"{rel}:{line}")
        for m in re.finditer(r'POPCORN_INSTANTIATE_KERNEL\("(\w+)",\s*(\w+)((?:,\s*[\w:]+)*)\)', text):
            names[m.group(1)] = (m.group(2), [a.strip() for a in m.group(3).split(",") if a.strip()])
    out = {}
    for name, (tmpl, targs) in sorted(names.items()):
        params, where = templates[tmpl]
        n = 0
        while n < len(params) and params[n][0] == "ptr":
            n += 1
        consts = []
        for kind, what in params[n:]:
            struct = what
            if struct not in sizes and targs:  # a template parameter naming the struct
                struct = targs[-1]
            consts.append(sizes[struct])
        out[name] = {"buffers": n, "constants": consts, "source": where}
    with open(os.path.join(os.path.dirname(os.path.abspath(__file__)), "reference_kernel_abi.json"), "w") as f:
        json.dump(out, f, indent=1, sort_keys=True)
        f.write("\n")
    print(f"{len(out)} kernels")


if __name__ == "__main__":
    main()
