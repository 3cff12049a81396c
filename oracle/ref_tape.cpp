// Writes a tape with the reference's own proto::TapeWriter
// (include/proto/tape.hpp:109-168) to argv[1], for the fixture
// tests/golden/tape_records.bin (tests/golden/make_tape.py runs it).  The
// records are the ones tests/cpp/test_tape.cpp writes with
// suf_hip::TapeWriter.  Built by oracle/build_ref.sh.  TEST INFRASTRUCTURE ONLY.
#include <span>       // tape.hpp uses std::span without including it
#include <stdexcept>  // and std::runtime_error
#include <vector>

#include "proto/tape.hpp"

int main(int argc, char** argv) {
  if (argc < 2) return 2;
  proto::FileTapeSink sink(argv[1]);
  proto::TapeWriter w(sink);
  w.write_u64(0x0123456789abcdefull);
  w.write_u64_vec(std::vector<proto::u64>{1, 2, 3, ~proto::u64(0)});
  w.write_bytes(std::vector<proto::u8>{'h', 'e', 'l', 'l', 'o'});
  w.write_bytes(std::vector<proto::u8>{});
  w.write_triple64(proto::Triple64Share{1, 2, 3});
  w.write_triple64_vec(std::vector<proto::Triple64Share>{{4, 5, 6}, {7, 8, 9}});
  w.write_u64(0);
  w.flush();
  return 0;
}
