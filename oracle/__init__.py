"""CPU oracle of Skyla's quantized weight path -- TEST INFRASTRUCTURE ONLY.

A restatement of the reference's f32 CPU path (skyla-gguf/src/quant.rs, skyla-ref/src/
{matrix,ffn,ops}.rs, moe_sort.comp) in C (skyla_oracle.c, loaded by skyla_oracle.py) and a
second, independent numpy restatement of the dequantisers (quant_np.py).

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may import or run
anything here, and only as the checker or the timed CPU baseline: the product library never
calls it, and no product path falls back to it.

The reference itself is Rust and cannot be built in this image (no cargo/rustc), so there is
no oracle/_ref build; see the parity notes at the top of each function's test.
"""
