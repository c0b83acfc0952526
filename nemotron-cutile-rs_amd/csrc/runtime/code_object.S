/* Embeds the gfx950 code object built from csrc/kernels/nh_kernels.hip into
 * libnemotron_hip.so; nh_context_create hands it to hipModuleLoadData. */
    .section .rodata.nh_code_object, "a", @progbits
    .balign 4096
    .globl nh_gfx950_code_object
    .type nh_gfx950_code_object, @object
nh_gfx950_code_object:
    .incbin NH_CODE_OBJECT
    .globl nh_gfx950_code_object_end
nh_gfx950_code_object_end:
    .byte 0
    .section .note.GNU-stack, "", @progbits
