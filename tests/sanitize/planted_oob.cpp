// A planted fault for tests/test_sanitize.py (CPU only, never part of the library):
// reads one element past a heap array, which the sanitized build must report. It shows
// that the harness running the library's tests under the sanitizers would catch such
// a read in the library's own host code.
#include <cstdlib>

extern "C" int dqsan_planted_oob(int n) {
  int* a = static_cast<int*>(std::calloc(static_cast<size_t>(n), sizeof(int)));
  const int v = a[n];  // one past the end
  std::free(a);
  return v;
}
