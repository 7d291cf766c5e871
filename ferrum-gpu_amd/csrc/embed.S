/* embed.S -- places the gfx950 FFT code object inside libferrum_gpu.so so the
 * HIP backend can hand it to hipModuleLoadData without touching the file
 * system (FG_HSACO_PATH is set by the Makefile). */
    .section .rodata.fg_fft_code_object,"a",@progbits
    .p2align 12
    .globl fg_fft_code_object_start
    .hidden fg_fft_code_object_start
fg_fft_code_object_start:
    .incbin FG_HSACO_PATH
    .globl fg_fft_code_object_end
    .hidden fg_fft_code_object_end
fg_fft_code_object_end:
    .byte 0
    .section .note.GNU-stack,"",@progbits
