/* The gfx950 code objects, linked into libskyla_hip.so and loaded with hipModuleLoadData.
   Built by skyla-kernel_amd/build.py, which puts the .hsaco files on the include path. */
#define EMBED(sym, file)            \
    .globl sym;                     \
    .globl sym##_end;               \
    .balign 4096;                   \
sym:                                \
    .incbin file;                   \
sym##_end:                          \
    .byte 0

    .section .rodata
EMBED(skyla_co_matvec, "matvec.hsaco")
EMBED(skyla_co_matmul, "matmul.hsaco")
EMBED(skyla_co_moe, "moe.hsaco")
EMBED(skyla_co_util, "util.hsaco")
EMBED(skyla_co_attention, "attention.hsaco")
    .section .note.GNU-stack,"",@progbits
