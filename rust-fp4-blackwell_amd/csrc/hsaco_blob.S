/* Embeds the gfx950 code object (kernels.hsaco) into the host library; the
 * runtime hands it to hipModuleLoadData at rfp4_init. */
    .section .rodata
    .global rfp4_hsaco_start
    .global rfp4_hsaco_end
    .balign 4096
rfp4_hsaco_start:
    .incbin "kernels.hsaco"
rfp4_hsaco_end:
    .byte 0
    .section .note.GNU-stack,"",@progbits
