// The gfx950 code objects built from kernels.hip and ingest.hip, linked into
// the library as read-only data and loaded with hipModuleLoadData at init.
    .section .rodata
    .balign 4096
    .global sml_code_object
    .type sml_code_object, @object
sml_code_object:
    .incbin "kernels.hsaco"
    .global sml_code_object_end
sml_code_object_end:
    .byte 0
    .balign 4096
    .global sml_ingest_object
    .type sml_ingest_object, @object
sml_ingest_object:
    .incbin "ingest.hsaco"
    .global sml_ingest_object_end
sml_ingest_object_end:
    .byte 0
    .section .note.GNU-stack,"",@progbits
