// Driver (test infrastructure) that runs the reference's FIDESlib-free
// headers, included from the reference tree, so that the library's own
// restatements can be compared with them:
//   native/fideslib_stage0/include/rotation_steps.hpp:11-47 (NAF steps)
//   native/fideslib_stage0/include/plaintext_rns.hpp:10-25 (compact bound)
// Reads commands on stdin, one per line, and prints one result per line:
//   naf V                -> steps...
//   rot OFFSET SLOTS NAF -> steps...   (or "error")
//   fits SLOTS SCALE Q V1 V2 ...       -> 0|1
#include "plaintext_rns.hpp"
#include "rotation_steps.hpp"

#include <cstdint>
#include <iostream>
#include <sstream>
#include <string>
#include <vector>

int main() {
  std::string line;
  while (std::getline(std::cin, line)) {
    std::istringstream in(line);
    std::string cmd;
    in >> cmd;
    try {
      if (cmd == "naf") {
        int v;
        in >> v;
        for (int s : fhemamba::naf_steps(v)) std::cout << s << ' ';
        std::cout << '\n';
      } else if (cmd == "rot") {
        int off, slots, naf;
        in >> off >> slots >> naf;
        for (int s : fhemamba::rotation_steps(off, slots, naf != 0)) std::cout << s << ' ';
        std::cout << '\n';
      } else if (cmd == "fits") {
        unsigned slots;
        double scale;
        unsigned long long q;
        in >> slots >> scale >> q;
        std::vector<double> vals;
        std::string tok;
        while (in >> tok) vals.push_back(std::stod(tok));
        std::cout << (fhemamba::compact_plaintext_fits(vals, slots, scale, q) ? 1 : 0) << '\n';
      } else {
        std::cout << "error\n";
      }
    } catch (const std::exception&) {
      std::cout << "error\n";
    }
  }
  return 0;
}
