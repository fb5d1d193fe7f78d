// Writes ark::host::lr_now (ark_amd/host/ark_host.hpp) for steps 0..N-1 to
// stdout as raw little-endian fp32, so a CPU test can compare the C++ mirror
// of optimizer.rs:80-92 with the Python one bit for bit.  Touches no GPU.
// Usage: lr_table <lr> <warmup_steps> <N>
#include <stdio.h>
#include <stdlib.h>

#include <vector>

#include "ark_host.hpp"

int main(int argc, char** argv) {
  if (argc != 4) {
    fprintf(stderr, "usage: lr_table <lr> <warmup_steps> <N>\n");
    return 2;
  }
  ark::host::AdamConfig cfg;
  cfg.lr = strtof(argv[1], nullptr);
  cfg.warmup_steps = (uint32_t)strtoul(argv[2], nullptr, 10);
  const uint32_t n = (uint32_t)strtoul(argv[3], nullptr, 10);
  std::vector<float> out(n);
  for (uint32_t s = 0; s < n; ++s) out[s] = ark::host::lr_now(cfg, s);
  return fwrite(out.data(), sizeof(float), n, stdout) == n ? 0 : 1;
}
