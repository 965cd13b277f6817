// Host build of the device's fp8 rounding (helix_runtime_amd/csrc/fp8.hpp,
// fp8_code is __host__ __device__): reads float32 values from argv[1] and
// writes one E4M3 code byte per value to argv[2].
#include "../../helix_runtime_amd/csrc/fp8.hpp"

#include <cstdio>

int main(int argc, char** argv) {
  if (argc != 3) return 2;
  std::FILE* in = std::fopen(argv[1], "rb");
  std::FILE* out = std::fopen(argv[2], "wb");
  if (in == nullptr || out == nullptr) return 3;
  float x = 0.0f;
  while (std::fread(&x, sizeof x, 1, in) == 1) {
    const auto c = static_cast<unsigned char>(helix::hip::fp8_code(x));
    std::fwrite(&c, 1, 1, out);
  }
  std::fclose(in);
  return std::fclose(out) == 0 ? 0 : 4;
}
