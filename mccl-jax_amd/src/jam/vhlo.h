// VHLO → jam IR: the operations, types and attributes of a StableHLO
// portable artifact (the MLIR bytecode jaxlib hands PJRT_Client_Compile).
//
// The reference turns the artifact back into StableHLO with the MLIR
// libraries (src/jam/parse.cc:53-63, deserializePortableArtifact, then the
// Normalize passes of parse.cc:33-50).  Here bytecode.cc reads the container
// and this file decodes what it holds:
//  - VHLO types (vhlo.tensor_v1, element types, vhlo.func_v1's function type),
//    by their binary type codes;
//  - the attributes the lowering reads (dimension lists, enums, integers,
//    booleans, strings, dense tensors, arrays, dictionaries), each read by the
//    shape its attribute name calls for and checked to consume its payload
//    exactly;
//  - the value numbering of MLIR bytecode (block arguments, then op results,
//    per region; isolated regions restart at zero, other nested regions
//    continue after their parent region's values);
//  - every `vhlo.<op>_v<N>` becomes `stablehlo.<op>` with the attributes in
//    the form the text reader gives them (dot, gather and scatter dimension
//    numbers regrouped into their dictionaries), vhlo.func_v1 a function,
//    vhlo.call_v1 a call and vhlo.return_v1 a return.
#pragma once

#include <memory>
#include <string>

#include "jam/bytecode.h"
#include "jam/ir.h"

namespace mi::jam {

// Builds the module an artifact encodes.  Returns nullptr and sets `error`
// ("jam: VHLO: ...") when something in it is malformed or not carried.
std::unique_ptr<Module> FromVhlo(const bytecode::Module& bm, std::string& error);

}  // namespace mi::jam
