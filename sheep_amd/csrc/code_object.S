// The gfx950 code object built from kernels.hip, linked into the library as
// read-only data and loaded with hipModuleLoadData at init.
    .section .rodata
    .balign 4096
    .global sml_code_object
    .type sml_code_object, @object
sml_code_object:
    .incbin "kernels.hsaco"
    .global sml_code_object_end
sml_code_object_end:
    .byte 0
    .section .note.GNU-stack,"",@progbits
