/* Embeds the gfx950 kernel code object (built from csrc/kernels/nk_all.hip) in the library. */
    .section .rodata
    .global nk_code_object_start
    .global nk_code_object_end
    .balign 4096
nk_code_object_start:
    .incbin NK_CODE_OBJECT
nk_code_object_end:
    .byte 0
    .section .note.GNU-stack,"",@progbits
