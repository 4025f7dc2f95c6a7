"""The ctypes mirrors of the C-ABI structs have the header's layout: a C
program built from include/ncmorph_amd.h prints every field's offset and
each struct's size, and the Python structures must agree."""
import ctypes as C
import os
import subprocess

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))

STRUCTS = {
    "ncm_decoder_shape_t": ("decoder", "_Shape"),
    "ncm_decoder_layer_t": ("decoder", "_Layer"),
    "ncm_decoder_layer_f32_t": ("decoder", "_LayerF32"),
    "ncm_decoder_trace_t": ("decoder", "_Trace"),
    "ncm_ncm_shape_t": ("ncm", "_Shape"),
    "ncm_ncm_weights_t": ("ncm", "_Weights"),
    "ncm_ncm_weights_f32_t": ("ncm", "_WeightsF32"),
    "ncm_vq_tok_t": ("vq_tokenizer", "_Tok"),
    "ncm_vq_tok_decoder_t": ("vq_tokenizer", "_Dec"),
}


def _c_layout(tmp_path):
    import importlib

    lines = ['#include <stdio.h>', '#include <stddef.h>', '#include "ncmorph_amd.h"',
             "int main(void) {"]
    for cname, (mod, cls) in STRUCTS.items():
        py = getattr(importlib.import_module(f"ncmorph_amd.{mod}"), cls)
        lines.append(f'printf("{cname} size %zu\\n", sizeof({cname}));')
        for f, _ in py._fields_:
            lines.append(f'printf("{cname} {f} %zu\\n", offsetof({cname}, {f}));')
    lines += ["return 0;", "}"]
    src = tmp_path / "layout.c"
    exe = tmp_path / "layout"
    src.write_text("\n".join(lines))
    subprocess.run(["gcc", "-std=c11", "-I", os.path.join(ROOT, "include"), str(src), "-o",
                    str(exe)], check=True)
    out = subprocess.run([str(exe)], check=True, capture_output=True, text=True).stdout
    return {tuple(l.split()[:2]): int(l.split()[2]) for l in out.splitlines()}


def test_struct_layouts_match_header(tmp_path):
    import importlib

    c = _c_layout(tmp_path)
    for cname, (mod, cls) in STRUCTS.items():
        py = getattr(importlib.import_module(f"ncmorph_amd.{mod}"), cls)
        assert C.sizeof(py) == c[(cname, "size")], cname
        for f, _ in py._fields_:
            assert getattr(py, f).offset == c[(cname, f)], (cname, f)
