/* codeobj.S — embeds the gfx950 code object (built by hipcc --genco) in the
 * library, so the shared object is self-contained. */
    .section .rodata
    .balign 4096
    .globl mynah_codeobj
    .type mynah_codeobj, @object
mynah_codeobj:
    .incbin "kernels.hsaco"
    .globl mynah_codeobj_end
mynah_codeobj_end:
    .byte 0
    .section .note.GNU-stack,"",@progbits
