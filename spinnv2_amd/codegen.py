"""Static C deployment wrappers for mi355x SPK packages.

The reference's codegen (compiler/codegen/c_codegen.py:98-136) embeds a
package in a C source with a small API (`<name>_init / _run / _run_checked /
_run_multi / _verify_checksum / _free`), a `main_test.c` that runs it on
files, and a build file.  The generated code here keeps that API and calls
libspkv2_mi355x instead of the CPU runtime:

  * the activation arena and the scratch arena are device memory, allocated
    by the runtime at `<name>_init` (the reference's static host arrays would
    not be reachable by the GPU);
  * `<name>_run*` take host buffers and copy them in and out
    (spkv2_set_input / spkv2_get_output), `<name>_run_device` binds
    device-resident buffers instead (spkv2_bind_input / _output, no copies);
  * with `external_weights` the package's weight section is zeroed in the
    embedded copy and patched back from a file at init; the loader's own
    checksum then verifies the restored weights.

A Makefile replaces the reference's CMakeLists.txt (gcc on the generated C,
linked against libspkv2_mi355x.so with an rpath).
"""

from __future__ import annotations

import re
from dataclasses import dataclass
from pathlib import Path

from .spk import format as F


@dataclass
class SpkInfo:
    input_sizes: list[int]
    output_sizes: list[int]
    weights_offset: int
    weights_size: int
    checksum: int          # FNV-1a-32 of the embedded bytes


def sanitize(name: str) -> str:
    s = re.sub(r"[^0-9A-Za-z_]", "_", name)
    return s if s and not s[0].isdigit() else f"m_{s}"


def inspect_spk(data: bytes) -> SpkInfo:
    """Input / output sizes in graph order (the metadata JSON's lists, the
    order the runtime indexes them by) and the weight section."""
    import json

    if len(data) < F.HEADER.size:
        raise ValueError("package smaller than its header")
    hdr = F.HEADER.unpack_from(data, 0)
    if hdr[0] != F.MAGIC:
        raise ValueError("not an SPK package")
    secs = {}
    for i in range(hdr[5]):
        s = F.SECTION.unpack_from(data, hdr[4] + i * F.SECTION.size)
        secs.setdefault(s[0], s)
    if F.SECTION_TENSOR_TABLE not in secs or F.SECTION_METADATA not in secs:
        raise ValueError("package lacks a tensor table or metadata")
    toff = secs[F.SECTION_TENSOR_TABLE][2]
    size = {i: F.TENSOR.unpack_from(data, toff + i * F.TENSOR.size)[13] for i in range(hdr[7])}
    m = secs[F.SECTION_METADATA]
    meta = json.loads(bytes(data[m[2]:m[2] + m[3]]).decode())
    ins = [int(size[t]) for t in meta["inputs"]]
    outs = [int(size[t]) for t in meta["outputs"]]
    if not ins or not outs:
        raise ValueError("package needs at least one input and one output")
    w = secs.get(F.SECTION_WEIGHTS, (0, 0, 0, 0))
    return SpkInfo(ins, outs, int(w[2]), int(w[3]), F.fnv1a32(data))


def _bytes_literal(data: bytes, per_line: int = 16) -> str:
    lines = []
    for i in range(0, len(data), per_line):
        lines.append("    " + ", ".join(f"0x{b:02x}" for b in data[i:i + per_line]) + ",")
    return "\n".join(lines) if lines else "    0x00,"


def header_text(sym: str, info: SpkInfo, external_weights: bool) -> str:
    S = sym.upper()
    macros = [f"#define {S}_INPUT_SIZE_{i} ((size_t){n}u)" for i, n in enumerate(info.input_sizes)]
    macros += [f"#define {S}_OUTPUT_SIZE_{i} ((size_t){n}u)" for i, n in enumerate(info.output_sizes)]
    macros += [f"#define {S}_INPUT_COUNT {len(info.input_sizes)}", f"#define {S}_OUTPUT_COUNT {len(info.output_sizes)}",
               f"#define {S}_INPUT_SIZE {S}_INPUT_SIZE_0", f"#define {S}_OUTPUT_SIZE {S}_OUTPUT_SIZE_0",
               f"#define {S}_SPK_CHECKSUM 0x{info.checksum:08x}u"]
    init = f"int {sym}_init(const char *weights_path);" if external_weights else f"int {sym}_init(void);"
    body = "\n".join(macros)
    return f"""/* Generated from an mi355x SPK package: runs it on the GPU through
 * libspkv2_mi355x.  Host buffers for _run / _run_checked / _run_multi,
 * device buffers for _run_device. */
#ifndef {S}_H
#define {S}_H

#include <stddef.h>

#ifdef __cplusplus
extern "C" {{
#endif

{body}

{init}
int {sym}_run(const void *input, void *output);
int {sym}_run_checked(const void *input, size_t input_size, void *output, size_t output_size);
int {sym}_run_multi(const void *const *inputs, const size_t *input_sizes, int num_inputs,
                    void *const *outputs, const size_t *output_sizes, int num_outputs);
int {sym}_run_device(void *const *device_inputs, int num_inputs, void *const *device_outputs, int num_outputs);
int {sym}_verify_checksum(const void *data, size_t size);
void {sym}_free(void);

#ifdef __cplusplus
}}
#endif

#endif /* {S}_H */
"""


def source_text(sym: str, blob: bytes, info: SpkInfo, external_weights: bool) -> str:
    S = sym.upper()
    qual = "" if external_weights else "const "
    if external_weights:
        init_sig = f"int {sym}_init(const char *weights_path)"
        patch = f"""    FILE *fp = fopen(weights_path, "rb");
    if (!fp) return -20;
    size_t got = fread(g_{sym}_spk + {info.weights_offset}u, 1, {info.weights_size}u, fp);
    int extra = fgetc(fp);
    fclose(fp);
    if (got != {info.weights_size}u || extra != EOF) return -21; /* not this package's weights */
"""
        # back to the shipped (zeroed) bytes, so a later init verifies again
        unpatch = f"    memset(g_{sym}_spk + {info.weights_offset}u, 0, {info.weights_size}u);\n"
    else:
        init_sig = f"int {sym}_init(void)"
        patch = unpatch = ""
    size_table_in = ", ".join(f"{S}_INPUT_SIZE_{i}" for i in range(len(info.input_sizes)))
    size_table_out = ", ".join(f"{S}_OUTPUT_SIZE_{i}" for i in range(len(info.output_sizes)))
    return f"""#include "{sym}.h"

#include "spkv2_runtime.h"

#include <stdint.h>
#include <stdio.h>
#include <string.h>

static {qual}unsigned char g_{sym}_spk[] __attribute__((aligned(64))) = {{
{_bytes_literal(blob)}
}};

static const size_t g_{sym}_in_sizes[] = {{{size_table_in}}};
static const size_t g_{sym}_out_sizes[] = {{{size_table_out}}};
static Spkv2Context *g_{sym}_ctx;

static uint32_t {sym}_fnv1a32(const unsigned char *data, size_t size) {{
    uint32_t value = 2166136261u;
    for (size_t i = 0; i < size; i++) {{
        value ^= data[i];
        value *= 16777619u;
    }}
    return value;
}}

int {sym}_verify_checksum(const void *data, size_t size) {{
    if (!data || size == 0) return -1;
    return {sym}_fnv1a32((const unsigned char *)data, size) == {S}_SPK_CHECKSUM ? 0 : -2;
}}

{init_sig} {{
    if (g_{sym}_ctx) return 0;
    if ({sym}_verify_checksum(g_{sym}_spk, sizeof(g_{sym}_spk)) != 0) return -10;
{patch}    int rc = spkv2_load_memory(g_{sym}_spk, sizeof(g_{sym}_spk), &g_{sym}_ctx);
    if (rc != 0) return rc;
    /* device arena and scratch: the runtime allocates both on the GPU */
    rc = spkv2_prepare(g_{sym}_ctx, NULL, 0);
    if (rc != 0) {{
        spkv2_free(g_{sym}_ctx);
        g_{sym}_ctx = 0;
    }}
    return rc;
}}

int {sym}_run_multi(const void *const *inputs, const size_t *input_sizes, int num_inputs,
                    void *const *outputs, const size_t *output_sizes, int num_outputs) {{
    if (!inputs || !outputs || !input_sizes || !output_sizes) return -1;
    if (num_inputs != {S}_INPUT_COUNT || num_outputs != {S}_OUTPUT_COUNT) return -2;
    if (!g_{sym}_ctx) return -3;
    for (int i = 0; i < num_inputs; i++) {{
        if (!inputs[i] || input_sizes[i] != g_{sym}_in_sizes[i]) return -2;
        int rc = spkv2_set_input(g_{sym}_ctx, i, inputs[i], input_sizes[i]);
        if (rc != 0) return rc;
    }}
    int rc = spkv2_run(g_{sym}_ctx);
    if (rc != 0) return rc;
    for (int i = 0; i < num_outputs; i++) {{
        if (!outputs[i] || output_sizes[i] != g_{sym}_out_sizes[i]) return -2;
        rc = spkv2_get_output(g_{sym}_ctx, i, outputs[i], output_sizes[i]);
        if (rc != 0) return rc;
    }}
    return 0;
}}

int {sym}_run_checked(const void *input, size_t input_size, void *output, size_t output_size) {{
    if (!input || !output) return -1;
    if ({S}_INPUT_COUNT != 1 || {S}_OUTPUT_COUNT != 1) return -2;
    if (input_size != {S}_INPUT_SIZE || output_size != {S}_OUTPUT_SIZE) return -2;
    return {sym}_run_multi(&input, &input_size, 1, &output, &output_size, 1);
}}

int {sym}_run(const void *input, void *output) {{
    return {sym}_run_checked(input, {S}_INPUT_SIZE, output, {S}_OUTPUT_SIZE);
}}

int {sym}_run_device(void *const *device_inputs, int num_inputs, void *const *device_outputs, int num_outputs) {{
    if (!device_inputs || !device_outputs) return -1;
    if (num_inputs != {S}_INPUT_COUNT || num_outputs != {S}_OUTPUT_COUNT) return -2;
    if (!g_{sym}_ctx) return -3;
    for (int i = 0; i < num_inputs; i++) {{
        int rc = spkv2_bind_input(g_{sym}_ctx, i, device_inputs[i], g_{sym}_in_sizes[i]);
        if (rc != 0) return rc;
    }}
    for (int i = 0; i < num_outputs; i++) {{
        int rc = spkv2_bind_output(g_{sym}_ctx, i, device_outputs[i], g_{sym}_out_sizes[i]);
        if (rc != 0) return rc;
    }}
    return spkv2_run(g_{sym}_ctx);
}}

void {sym}_free(void) {{
    spkv2_free(g_{sym}_ctx);
    g_{sym}_ctx = 0;
{unpatch}}}
"""


def main_test_text(sym: str, external_weights: bool) -> str:
    S = sym.upper()
    argc = 4 if external_weights else 3
    usage = "input.bin output.bin weights.bin" if external_weights else "input.bin output.bin"
    init = f"{sym}_init(argv[3])" if external_weights else f"{sym}_init()"
    return f"""#include "{sym}.h"

#include <stdio.h>
#include <stdlib.h>

static unsigned char *read_file(const char *path, size_t *out_size) {{
    FILE *fp = fopen(path, "rb");
    if (!fp) return NULL;
    fseek(fp, 0, SEEK_END);
    long size = ftell(fp);
    rewind(fp);
    if (size < 0) {{
        fclose(fp);
        return NULL;
    }}
    unsigned char *data = (unsigned char *)malloc(size > 0 ? (size_t)size : 1u);
    if (!data || fread(data, 1, (size_t)size, fp) != (size_t)size) {{
        free(data);
        fclose(fp);
        return NULL;
    }}
    fclose(fp);
    *out_size = (size_t)size;
    return data;
}}

int main(int argc, char **argv) {{
    if (argc != {argc}) {{
        fprintf(stderr, "usage: %s {usage}\\n", argv[0]);
        return 2;
    }}
    size_t in_size = 0;
    unsigned char *input = read_file(argv[1], &in_size);
    if (!input || in_size != {S}_INPUT_SIZE) {{
        fprintf(stderr, "input must be %zu bytes\\n", (size_t){S}_INPUT_SIZE);
        free(input);
        return 1;
    }}
    unsigned char *output = (unsigned char *)malloc({S}_OUTPUT_SIZE);
    int rc = {init};
    if (rc == 0) rc = {sym}_run(input, output);
    if (rc != 0) {{
        fprintf(stderr, "{sym} failed: %d\\n", rc);
        free(input);
        free(output);
        {sym}_free();
        return 1;
    }}
    FILE *fp = fopen(argv[2], "wb");
    int ok = fp && fwrite(output, 1, {S}_OUTPUT_SIZE, fp) == {S}_OUTPUT_SIZE;
    if (fp) fclose(fp);
    free(input);
    free(output);
    {sym}_free();
    return ok ? 0 : 1;
}}
"""


def makefile_text(sym: str, include_dir: Path, lib_dir: Path) -> str:
    return f"""# Builds the generated wrapper against libspkv2_mi355x (host C only; the
# GPU code lives in the runtime library).
INCLUDE ?= {include_dir}
LIBDIR ?= {lib_dir}
CFLAGS ?= -O2 -std=c11 -Wall -Wextra
LDFLAGS = -L$(LIBDIR) -lspkv2_mi355x -Wl,-rpath,$(LIBDIR)

all: lib{sym}.so {sym}_main_test

lib{sym}.so: {sym}.c {sym}.h
\t$(CC) $(CFLAGS) -fPIC -shared -I$(INCLUDE) {sym}.c -o $@ $(LDFLAGS)

{sym}_main_test: main_test.c {sym}.c {sym}.h
\t$(CC) $(CFLAGS) -I$(INCLUDE) main_test.c {sym}.c -o $@ $(LDFLAGS)

clean:
\trm -f lib{sym}.so {sym}_main_test
"""


def generate_c_from_spk(spk: bytes | str | Path, out_dir: str | Path, *, name: str = "model",
                        include_dir: str | Path | None = None, lib_dir: str | Path | None = None,
                        external_weights: bool = False) -> dict[str, Path]:
    """Writes <name>.h, <name>.c, main_test.c, Makefile (and, with
    `external_weights`, <name>_weights.bin) into out_dir; returns the paths."""
    data = bytes(spk) if isinstance(spk, (bytes, bytearray)) else Path(spk).read_bytes()
    sym = sanitize(name)
    info = inspect_spk(data)
    out = Path(out_dir)
    out.mkdir(parents=True, exist_ok=True)
    root = Path(__file__).resolve().parent
    include_dir = Path(include_dir) if include_dir else root.parent / "include"
    lib_dir = Path(lib_dir) if lib_dir else root / "lib"
    files = {}
    blob = data
    if external_weights and info.weights_size > 0:
        weights = data[info.weights_offset:info.weights_offset + info.weights_size]
        blob = bytearray(data)
        blob[info.weights_offset:info.weights_offset + info.weights_size] = bytes(info.weights_size)
        blob = bytes(blob)
        info.checksum = F.fnv1a32(blob)
        files["weights"] = out / f"{sym}_weights.bin"
        files["weights"].write_bytes(weights)
    ext = external_weights and info.weights_size > 0
    files["header"] = out / f"{sym}.h"
    files["header"].write_text(header_text(sym, info, ext))
    files["source"] = out / f"{sym}.c"
    files["source"].write_text(source_text(sym, blob, info, ext))
    files["main"] = out / "main_test.c"
    files["main"].write_text(main_test_text(sym, ext))
    files["makefile"] = out / "Makefile"
    files["makefile"].write_text(makefile_text(sym, include_dir.resolve(), lib_dir.resolve()))
    return files


EXAMPLE_DIR = Path(__file__).resolve().parent / "lib" / "codegen"


def build_examples() -> dict[str, Path]:
    """Generates and compiles the LeNet wrapper (embedded weights and
    external weights) under spinnv2_amd/lib/codegen/, next to the runtime
    library it links; the GPU tests load what this leaves there."""
    import subprocess

    from .spk import models, write_spk

    blob = write_spk(models.lenet(), "mi355x")
    out = {}
    for name, ext in (("lenet", False), ("lenet_ext", True)):
        d = EXAMPLE_DIR / name
        generate_c_from_spk(blob, d, name=name, external_weights=ext)
        subprocess.run(["make", "-s", "-B", "-C", str(d)], check=True)
        out[name] = d
    return out

