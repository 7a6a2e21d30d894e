// st_writer_ref.cpp — test infrastructure: writes a fixed set of tensors
// with the reference's SafeTensorsWriter (safetensors_writer.h, compiled
// from the reference sources by `make -C oracle ref`) so that the bytes of
// the library's writer can be compared with it.
//
//   st_writer_ref OUT.safetensors
#include <cstdint>
#include <cstdio>

#include "safetensors_writer.h"

int main(int argc, char** argv) {
    if (argc != 2) {
        fprintf(stderr, "usage: %s OUT.safetensors\n", argv[0]);
        return 2;
    }
    SafeTensorsWriter w;
    const int8_t q[6] = {0, 1, -2, 3, -128, 127};
    const float s[2] = {1.5f, -2.0f};
    const uint16_t b[1] = {0x3f80};
    const float z[1] = {3.25f};
    const uint8_t e[4] = {0x00, 0x38, 0xb8, 0x7e};
    w.add("transformer_blocks.0.attn.to_q.weight", "I8", {2, 3}, q, sizeof(q));
    w.add("transformer_blocks.0.attn.to_q.weight.__scales__", "F32", {2}, s, sizeof(s));
    w.add("quote\"name\\x", "BF16", {1}, b, sizeof(b));
    w.add("scalar", "F32", {}, z, sizeof(z));
    w.add("empty", "U8", {0}, nullptr, 0);
    w.add("e4m3", "F8_E4M3", {2, 2}, e, sizeof(e));
    return w.write(argv[1]) ? 0 : 1;
}
