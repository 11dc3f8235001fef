/* conv oracle: filled in with the implicit-GEMM convolution restatement */
