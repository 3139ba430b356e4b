// bundle_inspect.cpp -- test driver linked against the reference's own MIT2
// bundle loader (runtime/bundle.cpp, interface runtime/include/mit2/bundle.hpp:46-79).
// Test infrastructure only: it lets the bundle tests check that this
// project's loader accepts and rejects exactly the bundles the reference's
// loader does.
//
//   bundle_inspect PATH   ->  "OK <tensor count> <payload bytes>"  (exit 0)
//                             "ERR <message>"                      (exit 1)
#include <cstdio>
#include <exception>
#include <memory>

#include "mit2/bundle.hpp"

int main(int argc, char** argv) {
  if (argc != 2) {
    std::fprintf(stderr, "usage: %s BUNDLE\n", argv[0]);
    return 2;
  }
  try {
    mit2::Bundle b(argv[1]);
    std::printf("OK %zu %zu\n", b.tensor_count(), b.total_tensor_bytes());
    return 0;
  } catch (const std::exception& e) {
    std::printf("ERR %s\n", e.what());
    return 1;
  }
}
