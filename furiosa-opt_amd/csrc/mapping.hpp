// Mapping algebra for the MI355X backend: the `Mapping` value (MappingSerde JSON or `m![..]`
// text), its flattening into axis factors, and the resolver that turns a memory layout and a
// stream layout into the odometer wheels the HIP kernels walk.
//
// Reference semantics restated here (paths relative to the furiosa-opt repository):
//   * Mapping value and constructors   furiosa-mapping-types/src/lib.rs:144-337
//   * position semantics M::map         furiosa-mapping-types/src/dsl.rs:35-277
//   * m! grammar                        furiosa-mapping-macro/src/parser/parser.lalrpop:37-82
//   * sequence()/SequencerConfig        furiosa-mapping/src/lib.rs:107-116 (closed impl; restated from
//                                       docs/src/moving-tensors/sequencer.md:306-615)
//   * SequencerIter odometer            furiosa-mapping-types/src/lib.rs:875-988
//   * coalesce                          furiosa-mapping/src/lib.rs:184-203
//   * carve                             furiosa-mapping/src/lib.rs:154-167
//   * window_base                       furiosa-opt-std/src/storage/buf.rs:760-781
//
// A mapping is flattened (outer -> inner) into factors. A Term factor is one digit of one symbol:
// digit d in [0, extent) contributes d * weight to the symbol's coordinate, digits >= count are
// padding, and [weight, weight * period) is the span of the coordinate the digit owns. The
// sequencer splits every Term at the union of all span boundaries of its symbol (they must form a
// divisibility chain: the "compatible decompositions" rule of sequencer.md:589-615), so each stream
// piece reads exactly one memory piece, or none (a broadcast, stride 0).
#pragma once

#include <cstdint>
#include <map>
#include <memory>
#include <stdexcept>
#include <string>
#include <vector>

#include "json.hpp"

namespace fo::mapping {

struct Error : std::runtime_error {
  using std::runtime_error::runtime_error;
};

// Variant order follows lib.rs:563-573 (Bottom < Zero < Top).
enum class Pad : uint8_t { Bottom = 0, Zero = 1, Top = 2 };

struct Node;
using NodeP = std::shared_ptr<const Node>;

struct Node {
  enum Kind { Symbol, Stride, Modulo, Resize, Padding, Pair, Broadcast } kind;
  std::string sym;  // Symbol
  int64_t n = 0;    // Symbol size / stride / modulo / resize / padding extent / broadcast size
  Pad pad = Pad::Top;
  NodeP a, b;  // inner (a) or left (a) / right (b)
};

NodeP parse_json(const std::string& text);
NodeP from_json(const json::Value& v);
std::string to_json(const NodeP& m);
// `m![text]` with axis sizes (the `axes![..]` declaration).
NodeP parse_text(const std::string& text, const std::map<std::string, int64_t>& sizes);

int64_t size(const NodeP& m);
NodeP identity();
NodeP pair(const NodeP& l, const NodeP& r);  // Mapping::pair: drops an identity operand
std::vector<std::string> idents(const NodeP& m);

struct Factor {
  enum Kind { Term, Bcast, PadOnly } kind = Term;
  std::string sym;      // Term
  int64_t symsize = 0;  // Term: declared axis size
  int64_t weight = 1;   // Term: coordinate weight of one digit step
  int64_t period = 1;   // Term: the digit's span in coordinate space is [weight, weight*period)
  int64_t count = 1;    // live digits [0, count)
  int64_t extent = 1;   // wire extent; digits in [count, extent) are padding of kind `pad`
  Pad pad = Pad::Top;
};
using Factors = std::vector<Factor>;  // outer -> inner

Factors flatten(const NodeP& m);
NodeP unflatten(const Factors& f);
int64_t size(const Factors& f);
bool is_padding(const Factors& f);  // Mapping::is_padding: no live Symbol, no Broadcast > 1
// Mapping::remove_padding (furiosa-mapping-types/src/lib.rs:324-337): drops the padding of the left
// spine (leading pad-only factors, and the pad digits of the first live factor).
Factors remove_padding(const Factors& f);
// The first live axis term (outer -> inner) as a mapping of its own, unpadded (`axes().next()`
// then AxisTerm::to_term, as op_prep.rs:45-89 picks the indexed axis of scatter / gather).
Factors first_axis(const Factors& f);

// One odometer wheel, innermost-first in a Joint. `stride[k]` is the memory stride of memory k
// (0 = broadcast); digits >= `live` are padding of the stream.
struct Wheel {
  int64_t size = 1;
  int64_t live = 1;
  std::vector<int64_t> stride;
  int part = 0;  // which stream part (0 = outermost part) the wheel came from
};

struct Joint {
  std::vector<Wheel> wheels;  // innermost-first
  int64_t stream_size = 1;
  int64_t part_size(int part) const;
};

enum class Mode { Read, Write, Carve };

// Resolve the memories against a stream made of `parts` (outer -> inner, paired). Wheels never
// coalesce across a part boundary, so a part's wheels stay a contiguous run. Throws Error on an
// incompatible decomposition, a composite factor, or (unless `lenient`) an unconsumed memory.
Joint sequence(const std::vector<Factors>& memories, const std::vector<Factors>& parts, Mode mode,
               bool coalesce = true);

// MappingExt::carve: `self` with every piece `piece` backs replaced by a Top pad of its size.
Factors carve(const Factors& self, const Factors& piece);

// Dense wire offsets of each factor (product of the extents inside it).
std::vector<int64_t> strides(const Factors& f);

// window_base: the wire position of the live cell of `base` whose coordinates equal `coords`
// (symbols absent from `coords` are at 0; symbols absent from `base` are ignored).
int64_t window_base(const Factors& base, const std::map<std::string, int64_t>& coords);

// The symbols whose axis terms appear in `dst` but not in `src` (op_prep.rs:31-41).
std::vector<std::string> broadcast_symbols(const Factors& src, const Factors& dst);

std::map<std::string, int64_t> parse_offset_json(const std::string& text);

}  // namespace fo::mapping
