// VmProgram XML (VmProgramXml.cs) and the HIP program artifact
// (D3D12VmArtifact.cs:90-148) for HipVmProgram.
#include "si_graph.hpp"
#include "si_host.hpp"

#include <algorithm>
#include <array>
#include <cctype>
#include <cstdio>
#include <cstring>
#include <tuple>
#include <map>
#include <functional>
#include <set>
#include <sstream>

namespace sharpinference {
namespace {

// ---- a small XML element tree --------------------------------------------------------------

struct XElement {
    std::string name;
    std::vector<std::pair<std::string, std::string>> attributes;
    std::vector<XElement> children;

    XElement& Attr(const std::string& n, const std::string& v)
    {
        attributes.emplace_back(n, v);
        return *this;
    }
    XElement& Add(XElement e)
    {
        children.push_back(std::move(e));
        return children.back();
    }
    const std::string* Attribute(const std::string& n) const
    {
        for (const auto& a : attributes)
            if (a.first == n)
                return &a.second;
        return nullptr;
    }
};

XElement El(const std::string& name) { return XElement{name, {}, {}}; }

void Escape(std::string& out, const std::string& v)
{
    for (const char c : v) {
        switch (c) {
        case '&': out += "&amp;"; break;
        case '<': out += "&lt;"; break;
        case '>': out += "&gt;"; break;
        case '"': out += "&quot;"; break;
        case '\n': out += "&#xA;"; break;
        case '\r': out += "&#xD;"; break;
        case '\t': out += "&#x9;"; break;
        default: out += c;
        }
    }
}

// Two-space indentation, " />" for empty elements (XElement.ToString's form).
void Write(std::string& out, const XElement& e, int depth)
{
    out.append(static_cast<size_t>(2 * depth), ' ');
    out += '<';
    out += e.name;
    for (const auto& a : e.attributes) {
        out += ' ';
        out += a.first;
        out += "=\"";
        Escape(out, a.second);
        out += '"';
    }
    if (e.children.empty()) {
        out += " />";
        return;
    }
    out += '>';
    for (const auto& c : e.children) {
        out += '\n';
        Write(out, c, depth + 1);
    }
    out += '\n';
    out.append(static_cast<size_t>(2 * depth), ' ');
    out += "</";
    out += e.name;
    out += '>';
}

[[noreturn]] void Bad(const std::string& why) { throw InvalidDataException(why); }

// A restricted XML reader: elements, attributes, whitespace, comments and
// processing instructions (ignored); no DTD, no CDATA, no namespaces, no
// text.  Limits as XmlReaderSettings + the probe of VmProgramXml.cs:46-62.
class XmlReader {
public:
    explicit XmlReader(const std::string& s) : s_(s) {}

    XElement Document()
    {
        if (s_.size() > 16u * 1024 * 1024)
            Bad("Invalid VM program XML.");
        if (s_.size() >= 3 && static_cast<unsigned char>(s_[0]) == 0xEF && static_cast<unsigned char>(s_[1]) == 0xBB &&
            static_cast<unsigned char>(s_[2]) == 0xBF)
            i_ = 3;   // UTF-8 byte order mark
        Misc();
        if (i_ >= s_.size() || s_[i_] != '<')
            Bad("Invalid VM program XML.");
        XElement root = Element(0);
        Misc();
        if (i_ != s_.size())
            Bad("Invalid VM program XML.");
        return root;
    }

private:
    const std::string& s_;
    size_t i_ = 0;
    int elements_ = 0;

    bool Starts(const char* t) const { return s_.compare(i_, std::strlen(t), t) == 0; }
    static bool Space(char c) { return c == ' ' || c == '\t' || c == '\r' || c == '\n'; }
    void Skip()
    {
        while (i_ < s_.size() && Space(s_[i_]))
            i_++;
    }
    // whitespace, comments and processing instructions between elements
    void Misc()
    {
        for (;;) {
            Skip();
            if (Starts("<!--")) {
                const size_t e = s_.find("-->", i_ + 4);
                if (e == std::string::npos)
                    Bad("Invalid VM program XML.");
                i_ = e + 3;
            } else if (Starts("<?")) {
                const size_t e = s_.find("?>", i_ + 2);
                if (e == std::string::npos)
                    Bad("Invalid VM program XML.");
                i_ = e + 2;
            } else if (Starts("<!")) {
                Bad("Invalid VM program XML.");   // DTD (prohibited) or CDATA (text)
            } else {
                return;
            }
        }
    }
    std::string Name()
    {
        const size_t b = i_;
        while (i_ < s_.size() && (std::isalnum(static_cast<unsigned char>(s_[i_])) || s_[i_] == '_' || s_[i_] == '-' ||
                                  s_[i_] == '.' || s_[i_] == ':'))
            i_++;
        if (i_ == b || std::isdigit(static_cast<unsigned char>(s_[b])) || s_[b] == '-' || s_[b] == '.')
            Bad("Invalid VM program XML.");
        return s_.substr(b, i_ - b);
    }
    std::string Value(char quote)
    {
        std::string v;
        while (i_ < s_.size() && s_[i_] != quote) {
            const char c = s_[i_];
            if (c == '<')
                Bad("Invalid VM program XML.");
            if (c != '&') {
                v += c;
                i_++;
                continue;
            }
            const size_t e = s_.find(';', i_);
            if (e == std::string::npos || e - i_ > 12)
                Bad("Invalid VM program XML.");
            const std::string ent = s_.substr(i_ + 1, e - i_ - 1);
            i_ = e + 1;
            if (ent == "lt") v += '<';
            else if (ent == "gt") v += '>';
            else if (ent == "amp") v += '&';
            else if (ent == "quot") v += '"';
            else if (ent == "apos") v += '\'';
            else if (ent.size() > 1 && ent[0] == '#') {
                unsigned long code = 0;
                try {
                    size_t used = 0;
                    code = ent[1] == 'x' ? std::stoul(ent.substr(2), &used, 16) : std::stoul(ent.substr(1), &used, 10);
                    if (used != ent.size() - (ent[1] == 'x' ? 2 : 1))
                        Bad("Invalid VM program XML.");
                } catch (const std::logic_error&) {
                    Bad("Invalid VM program XML.");
                }
                if (code == 0 || code > 0x10FFFF)
                    Bad("Invalid VM program XML.");
                // UTF-8
                if (code < 0x80) {
                    v += static_cast<char>(code);
                } else if (code < 0x800) {
                    v += static_cast<char>(0xC0 | (code >> 6));
                    v += static_cast<char>(0x80 | (code & 0x3F));
                } else if (code < 0x10000) {
                    v += static_cast<char>(0xE0 | (code >> 12));
                    v += static_cast<char>(0x80 | ((code >> 6) & 0x3F));
                    v += static_cast<char>(0x80 | (code & 0x3F));
                } else {
                    v += static_cast<char>(0xF0 | (code >> 18));
                    v += static_cast<char>(0x80 | ((code >> 12) & 0x3F));
                    v += static_cast<char>(0x80 | ((code >> 6) & 0x3F));
                    v += static_cast<char>(0x80 | (code & 0x3F));
                }
            } else {
                Bad("Invalid VM program XML.");   // undeclared entity
            }
        }
        if (i_ >= s_.size())
            Bad("Invalid VM program XML.");
        i_++;   // closing quote
        return v;
    }
    XElement Element(int depth)
    {
        if (++elements_ > 100000 || depth > 64)
            Bad("VM XML exceeds element or nesting limits.");
        i_++;   // '<'
        XElement e = El(Name());
        for (;;) {
            const size_t before = i_;
            Skip();
            if (i_ >= s_.size())
                Bad("Invalid VM program XML.");
            if (s_[i_] == '/') {
                if (!Starts("/>"))
                    Bad("Invalid VM program XML.");
                i_ += 2;
                return e;
            }
            if (s_[i_] == '>') {
                i_++;
                break;
            }
            if (i_ == before)
                Bad("Invalid VM program XML.");   // attributes are separated by whitespace
            const std::string n = Name();
            Skip();
            if (i_ >= s_.size() || s_[i_] != '=')
                Bad("Invalid VM program XML.");
            i_++;
            Skip();
            if (i_ >= s_.size() || (s_[i_] != '"' && s_[i_] != '\''))
                Bad("Invalid VM program XML.");
            const char q = s_[i_++];
            std::string v = Value(q);
            if (e.Attribute(n))
                Bad("Invalid VM program XML.");   // duplicate attribute
            e.attributes.emplace_back(n, std::move(v));
        }
        for (;;) {
            Misc();
            if (i_ >= s_.size())
                Bad("Invalid VM program XML.");
            if (Starts("</")) {
                i_ += 2;
                if (Name() != e.name)
                    Bad("Invalid VM program XML.");
                Skip();
                if (i_ >= s_.size() || s_[i_] != '>')
                    Bad("Invalid VM program XML.");
                i_++;
                return e;
            }
            if (s_[i_] != '<')
                Bad("Unexpected XML content in '" + e.name + "'.");   // text content
            e.children.push_back(Element(depth + 1));
        }
    }
};

// ---- the reader's structural rules (VmProgramXml.cs:274-315) -------------------------------

void Check(const XElement& e, const char* name, std::initializer_list<const char*> attributes,
           std::initializer_list<const char*> children)
{
    const auto in = [](const std::string& v, std::initializer_list<const char*> set) {
        for (const char* x : set)
            if (v == x)
                return true;
        return false;
    };
    bool ok = e.name == name;
    for (const auto& a : e.attributes)
        ok = ok && a.first.find(':') == std::string::npos && a.first != "xmlns" && in(a.first, attributes);
    for (const auto& c : e.children)
        ok = ok && c.name.find(':') == std::string::npos && in(c.name, children);
    if (!ok)
        Bad(std::string("Unexpected XML content in '") + name + "'.");
}

const XElement* OptionalOne(const XElement& parent, const char* name)
{
    const XElement* found = nullptr;
    for (const auto& c : parent.children)
        if (c.name == name) {
            if (found)
                Bad(std::string("Duplicate '") + name + "'.");
            found = &c;
        }
    return found;
}

const XElement& One(const XElement& parent, const char* name)
{
    const XElement* e = OptionalOne(parent, name);
    if (!e)
        Bad(std::string("Missing '") + name + "'.");
    return *e;
}

const std::vector<XElement>& Container(const XElement& parent, const char* name, const char* child)
{
    const XElement& e = One(parent, name);
    Check(e, name, {}, {child});
    return e.children;
}

const std::string& Required(const XElement& e, const char* attribute)
{
    const std::string* v = e.Attribute(attribute);
    if (!v)
        Bad(std::string("Missing '") + attribute + "'.");
    return *v;
}

int64_t Integer(const XElement& e, const char* attribute, bool allow_sign)
{
    const std::string& v = Required(e, attribute);
    size_t i = 0;
    bool neg = false;
    if (allow_sign && !v.empty() && (v[0] == '-' || v[0] == '+')) {
        neg = v[0] == '-';
        i = 1;
    }
    if (i >= v.size())
        Bad("Invalid VM program XML.");
    uint64_t x = 0;
    for (; i < v.size(); i++) {
        if (!std::isdigit(static_cast<unsigned char>(v[i])))
            Bad("Invalid VM program XML.");
        const uint64_t next = x * 10 + static_cast<uint64_t>(v[i] - '0');
        if (next / 10 != x)
            Bad("Invalid VM program XML.");
        x = next;
    }
    if (allow_sign && x > static_cast<uint64_t>(INT32_MAX) + (neg ? 1 : 0))
        Bad("Invalid VM program XML.");
    return neg ? -static_cast<int64_t>(x) : static_cast<int64_t>(x);
}

template <typename E, size_t N>
E EnumValue(const XElement& e, const char* attribute, const std::array<const char*, N>& names)
{
    const std::string& v = Required(e, attribute);
    for (size_t i = 0; i < N; i++)
        if (v == names[i])
            return static_cast<E>(i);
    Bad(std::string("Invalid '") + attribute + "' value '" + v + "'.");
}

const std::array<const char*, 5> kElementTypes{"Byte", "Int32", "UInt32", "Float16", "Float32"};
const std::array<const char*, 3> kScopes{"Global", "Session", "Local"};
const std::array<const char*, 2> kVmAccess{"ReadOnly", "ReadWrite"};
const std::array<const char*, 3> kResourceAccess{"Read", "Write", "ReadWrite"};
const std::array<const char*, 3> kDefinitionKinds{"Function", "Kernel", "Orchestration"};
constexpr int kKernel = 1;
constexpr int kOrchestration = 2;
const char* kTarget = "Hip";
const char* kExecutionTarget = "hip.gfx950";

XElement Tensor(const TensorDescriptor& t)
{
    XElement e = El("Tensor");
    e.Attr("elementType", kElementTypes[static_cast<size_t>(t.element_type)]);
    for (const int64_t d : t.dimensions)
        e.Add(El("Dimension")).Attr("size", std::to_string(d));
    return e;
}

TensorDescriptor ReadTensor(const XElement& e)
{
    Check(e, "Tensor", {"elementType"}, {"Dimension"});
    TensorDescriptor t;
    t.element_type = EnumValue<GraphElementType>(e, "elementType", kElementTypes);
    for (const auto& d : e.children) {
        Check(d, "Dimension", {"size"}, {});
        const int64_t v = Integer(d, "size", true);
        if (v <= 0)
            Bad("A tensor requires positive dimensions.");
        t.dimensions.push_back(v);
    }
    if (t.dimensions.empty())
        Bad("A tensor requires positive dimensions.");
    return t;
}

XElement Arguments(const std::vector<std::tuple<std::string, std::string, uint64_t>>& args)
{
    XElement e = El("Arguments");
    for (const auto& [parameter, source, offset] : args)
        e.Add(El("Argument")).Attr("parameter", parameter).Attr("source", source).Attr("byteOffset", std::to_string(offset));
    return e;
}

struct Arg {
    std::string parameter, source;
    uint64_t offset;
};

std::vector<Arg> ReadArguments(const XElement& owner)
{
    std::vector<Arg> out;
    for (const auto& a : Container(owner, "Arguments", "Argument")) {
        Check(a, "Argument", {"parameter", "source", "byteOffset"}, {});
        out.push_back({Required(a, "parameter"), Required(a, "source"),
                       static_cast<uint64_t>(Integer(a, "byteOffset", false))});
    }
    return out;
}

bool SameTensor(const TensorDescriptor& a, const TensorDescriptor& b)
{
    return a.element_type == b.element_type && a.dimensions == b.dimensions;
}

}  // namespace

// ---- serialize -----------------------------------------------------------------------------

std::string SerializeVmProgram(const HipVmProgram& program)
{
    XElement root = El("VmProgram");
    root.Attr("name", program.name).Attr("abi", program.abi).Attr("target", kTarget);
    XElement& slots = root.Add(El("Slots"));
    for (const auto& s : program.Slots()) {
        XElement& e = slots.Add(El("Slot"));
        e.Attr("id", s.id).Attr("scope", kScopes[static_cast<size_t>(s.scope)]);
        e.Attr("access", kVmAccess[static_cast<size_t>(s.access)]);
        if (!s.binding_key.empty())
            e.Attr("bindingKey", s.binding_key);
        e.Add(Tensor(s.tensor));
    }
    XElement& state = root.Add(El("State"));
    state.Attr("schema", program.state_schema).Attr("version", std::to_string(program.state_version));
    for (const auto& s : program.state)
        state.Add(El("Entry")).Attr("name", s.name).Attr("slot", s.slot);
    XElement& definitions = root.Add(El("Definitions"));
    std::set<std::string> kernels;   // kernel definitions written so far
    XElement entries = El("Entries");
    for (const auto& [entry, dispatches] : program.Entries()) {
        // the entry's distinct slot views become definition parameters
        struct View {
            std::string name, slot;
            uint64_t offset;
            TensorDescriptor tensor;
            bool writes;
        };
        std::vector<View> views;
        std::set<std::string> taken;
        for (const auto& s : program.Slots())
            taken.insert(s.id);
        const auto view_of = [&](const InstructionParameter& p) -> View& {
            for (auto& v : views)
                if (v.slot == p.source && v.offset == p.byte_offset && SameTensor(v.tensor, p.tensor))
                    return v;
            const HipVmSlot& slot = program.Slots()[program.SlotIndex(p.source)];
            std::string name;
            if (p.byte_offset == 0 && SameTensor(slot.tensor, p.tensor)) {
                name = slot.id;
            } else {
                name = p.name;
                for (int k = 1; taken.count(name); k++)
                    name = p.source + "." + std::to_string(p.byte_offset) + "." + std::to_string(k);
                taken.insert(name);
            }
            views.push_back({name, p.source, p.byte_offset, p.tensor, false});
            return views.back();
        };
        XElement nodes = El("Nodes");
        int index = 0;
        for (const auto& d : dispatches) {
            const Instruction& ins = *d.instruction;
            std::vector<std::tuple<std::string, std::string, uint64_t>> args;
            std::vector<std::pair<std::string, std::string>> attributes, accesses;
            std::vector<std::string> writes;
            for (const auto& p : d.recording.parameters) {
                if (p.kind == InstructionParameter::Kind::Attribute) {
                    attributes.emplace_back(p.name, p.value);
                    continue;
                }
                View& v = view_of(p);
                const bool w = p.access != GraphResourceAccess::Read;
                v.writes = v.writes || w;
                args.emplace_back(p.name, v.name, 0);
                accesses.emplace_back(p.name, kResourceAccess[static_cast<size_t>(p.access)]);
                if (w && std::find(writes.begin(), writes.end(), v.name) == writes.end())
                    writes.push_back(v.name);
            }
            std::sort(attributes.begin(), attributes.end());
            std::sort(accesses.begin(), accesses.end());
            const std::string id = "dispatch_" + std::to_string(index);
            XElement& node = nodes.Add(El("Node"));
            node.Attr("id", id);
            node.Add(El("Dependencies"));
            // a lowered dispatch: the operator lives in its kernel definition
            // (one per distinct operator), bound to the definition's parameters,
            // and the orchestration dispatches it with its grid
            XElement kernel_body = El("Operator");
            const bool lowered = !d.launch.definition.empty();
            XElement& op = lowered ? kernel_body : node.Add(El("Operator"));
            if (lowered) {
                std::vector<std::tuple<std::string, std::string, uint64_t>> ports;
                for (const auto& [port, view, offset] : args)
                    ports.emplace_back(port, port, offset);
                XElement& dispatch = node.Add(El("Dispatch"));
                dispatch.Attr("definition", d.launch.definition);
                dispatch.Add(Arguments(args));
                dispatch.Add(El("Groups"))
                    .Attr("x", std::to_string(d.launch.groups[0]))
                    .Attr("y", std::to_string(d.launch.groups[1]))
                    .Attr("z", std::to_string(d.launch.groups[2]));
                args = ports;
            }
            op.Attr("name", ins.Name()).Attr("collection", ins.CollectionId());
            op.Add(Arguments(args));
            op.Add(El("Precision"))
                .Attr("minimumArithmeticType", kElementTypes[static_cast<size_t>(d.precision.minimum_arithmetic_type)])
                .Attr("minimumAccumulatorType", kElementTypes[static_cast<size_t>(d.precision.minimum_accumulator_type)]);
            op.Add(El("ResolvedPrecision"))
                .Attr("arithmeticType", kElementTypes[static_cast<size_t>(d.resolved.arithmetic_type)])
                .Attr("accumulatorType", kElementTypes[static_cast<size_t>(d.resolved.accumulator_type)]);
            op.Add(El("ExecutionConfiguration")).Attr("target", kExecutionTarget).Attr("implementation",
                                                                                        d.recording.operation);
            XElement& attrs = op.Add(El("Attributes"));
            for (const auto& [n, v] : attributes)
                attrs.Add(El("Attribute")).Attr("name", n).Attr("value", v);
            op.Add(El("IndexBounds"));
            XElement& ports = op.Add(El("ParameterAccesses"));
            for (const auto& [n, a] : accesses)
                ports.Add(El("Port")).Attr("name", n).Attr("access", a);
            if (lowered && kernels.insert(d.launch.definition).second) {
                XElement& kd = definitions.Add(El("Definition"));
                kd.Attr("id", d.launch.definition).Attr("kind", kDefinitionKinds[kKernel]);
                kd.Add(El("Threads")).Attr("x", std::to_string(d.launch.threads)).Attr("y", "1").Attr("z", "1");
                XElement& kp = kd.Add(El("Parameters"));
                for (const auto& prm : d.recording.parameters)
                    if (prm.kind == InstructionParameter::Kind::Tensor) {
                        XElement& pe = kp.Add(El("Parameter"));
                        pe.Attr("name", prm.name)
                            .Attr("access", prm.access != GraphResourceAccess::Read ? "ReadWrite" : "ReadOnly");
                        pe.Add(Tensor(prm.tensor));
                    }
                XElement& body = kd.Add(El("Nodes")).Add(El("Node"));
                body.Attr("id", "body");
                body.Add(El("Dependencies"));
                body.Add(std::move(kernel_body));
            }
            XElement& barrier = nodes.Add(El("Node"));
            barrier.Attr("id", "barrier_" + std::to_string(index));
            barrier.Add(El("Dependencies")).Add(El("NodeRef")).Attr("id", id);
            XElement& b = barrier.Add(El("Barrier"));
            for (const auto& w : writes)
                b.Add(El("Resource")).Attr("parameter", w);
            index++;
        }
        XElement& def = definitions.Add(El("Definition"));
        def.Attr("id", entry).Attr("kind", kDefinitionKinds[kOrchestration]);
        XElement& params = def.Add(El("Parameters"));
        std::vector<std::tuple<std::string, std::string, uint64_t>> bindings;
        for (const auto& v : views) {
            XElement& pe = params.Add(El("Parameter"));
            pe.Attr("name", v.name).Attr("access", v.writes ? "ReadWrite" : "ReadOnly");
            pe.Add(Tensor(v.tensor));
            bindings.emplace_back(v.name, v.slot, v.offset);
        }
        def.Add(std::move(nodes));
        XElement& en = entries.Add(El("Entry"));
        en.Attr("name", entry).Attr("definition", entry);
        en.Add(Arguments(bindings));
    }
    root.Add(std::move(entries));
    std::string out;
    Write(out, root, 0);
    return out;
}

// ---- deserialize ---------------------------------------------------------------------------

HipVmProgram DeserializeVmProgram(const std::string& xml, const std::shared_ptr<const InstructionRegistry>& registry_in)
{
    const auto registry = registry_in ? registry_in : DefaultHipRegistry();
    const XElement root = XmlReader(xml).Document();
    Check(root, "VmProgram", {"name", "abi", "target"}, {"Slots", "State", "Definitions", "Entries"});
    if (Required(root, "target") != kTarget)
        Bad("Invalid 'target' value '" + Required(root, "target") + "'.");
    HipVmProgram p;
    p.name = Required(root, "name");
    p.abi = Required(root, "abi");
    for (const auto& s : Container(root, "Slots", "Slot")) {
        Check(s, "Slot", {"id", "scope", "access", "bindingKey"}, {"Tensor"});
        HipVmSlot slot;
        slot.id = Required(s, "id");
        slot.scope = EnumValue<VmSlotScope>(s, "scope", kScopes);
        slot.access = EnumValue<VmAccess>(s, "access", kVmAccess);
        slot.tensor = ReadTensor(One(s, "Tensor"));
        if (const std::string* k = s.Attribute("bindingKey"))
            slot.binding_key = *k;
        p.AddSlot(std::move(slot));
    }
    const XElement& state = One(root, "State");
    Check(state, "State", {"schema", "version"}, {"Entry"});
    p.state_schema = Required(state, "schema");
    p.state_version = static_cast<int>(Integer(state, "version", true));
    for (const auto& e : state.children) {
        Check(e, "Entry", {"name", "slot"}, {});
        if (p.SlotIndex(Required(e, "slot")) < 0)
            Bad("State entry '" + Required(e, "name") + "' names an unknown slot.");
        p.state.push_back({Required(e, "name"), Required(e, "slot")});
    }
    struct Parameter {
        VmAccess access;
        TensorDescriptor tensor;
    };
    struct Definition {
        int kind;
        std::map<std::string, Parameter> parameters;
        const XElement* nodes;
        uint32_t threads = 0;
    };
    std::map<std::string, Definition> definitions;
    for (const auto& d : Container(root, "Definitions", "Definition")) {
        Check(d, "Definition", {"id", "kind"}, {"Threads", "Parameters", "Nodes"});
        Definition def{static_cast<int>(EnumValue<int>(d, "kind", kDefinitionKinds)), {}, &One(d, "Nodes"), 0};
        if (const XElement* threads = OptionalOne(d, "Threads")) {
            Check(*threads, "Threads", {"x", "y", "z"}, {});
            def.threads = static_cast<uint32_t>(Integer(*threads, "x", true));
            Integer(*threads, "y", true);
            Integer(*threads, "z", true);
        }
        for (const auto& pe : Container(d, "Parameters", "Parameter")) {
            Check(pe, "Parameter", {"name", "access"}, {"Tensor"});
            if (!def.parameters
                     .emplace(Required(pe, "name"),
                              Parameter{EnumValue<VmAccess>(pe, "access", kVmAccess), ReadTensor(One(pe, "Tensor"))})
                     .second)
                Bad("Duplicate definition parameter '" + Required(pe, "name") + "'.");
        }
        Check(*def.nodes, "Nodes", {}, {"Node"});
        if (!definitions.emplace(Required(d, "id"), std::move(def)).second)
            Bad("Duplicate definition '" + Required(d, "id") + "'.");
    }
    for (const auto& en : Container(root, "Entries", "Entry")) {
        Check(en, "Entry", {"name", "definition"}, {"Arguments"});
        const std::string& entry = Required(en, "name");
        const auto dit = definitions.find(Required(en, "definition"));
        if (dit == definitions.end())
            Bad("Entry '" + entry + "' names an unknown definition.");
        const Definition& def = dit->second;
        if (def.kind != kOrchestration)
            throw NotSupportedException("Entry '" + entry + "': the HIP executor runs orchestration definitions.");
        std::map<std::string, std::pair<std::string, uint64_t>> bound;   // parameter -> (slot, offset)
        for (const auto& a : ReadArguments(en)) {
            if (!def.parameters.count(a.parameter))
                Bad("Entry '" + entry + "' binds an unknown parameter '" + a.parameter + "'.");
            if (!bound.emplace(a.parameter, std::make_pair(a.source, a.offset)).second)
                Bad("Entry '" + entry + "' binds '" + a.parameter + "' twice.");
        }
        for (const auto& node : def.nodes->children) {
            Check(node, "Node", {"id"}, {"Dependencies", "Operator", "Call", "Dispatch", "Barrier"});
            Required(node, "id");
            for (const auto& r : Container(node, "Dependencies", "NodeRef")) {
                Check(r, "NodeRef", {"id"}, {});
                Required(r, "id");
            }
            const XElement* ins = nullptr;
            for (const auto& c : node.children)
                if (c.name != "Dependencies") {
                    if (ins)
                        Bad("A node must contain exactly one instruction.");
                    ins = &c;
                }
            if (!ins)
                Bad("A node must contain exactly one instruction.");
            if (ins->name == "Barrier") {
                Check(*ins, "Barrier", {}, {"Resource"});
                for (const auto& r : ins->children) {
                    Check(r, "Resource", {"parameter"}, {});
                    Required(r, "parameter");
                }
                continue;   // every dispatch of a HIP plan is ordered after the previous one
            }
            // where a name bound by the operator's arguments lives: (tensor, access, slot, byte offset)
            struct Bound {
                TensorDescriptor tensor;
                VmAccess access;
                std::string slot;
                uint64_t offset;
            };
            const auto orchestration_argument = [&](const std::string& name) -> Bound {
                const auto pit = def.parameters.find(name);
                const auto bit = bound.find(name);
                if (pit == def.parameters.end() || bit == bound.end())
                    Bad("Argument names an unbound parameter '" + name + "'.");
                return {pit->second.tensor, pit->second.access, bit->second.first, bit->second.second};
            };
            HipVmKernelLaunch launch;
            const XElement* op = ins;
            std::function<Bound(const std::string&)> resolve = orchestration_argument;
            std::map<std::string, Bound> kernel_bound;
            if (ins->name == "Dispatch") {
                Check(*ins, "Dispatch", {"definition"}, {"Arguments", "Groups"});
                launch.definition = Required(*ins, "definition");
                const auto kit = definitions.find(launch.definition);
                if (kit == definitions.end() || kit->second.kind != kKernel)
                    Bad("Dispatch names an unknown kernel definition '" + launch.definition + "'.");
                const Definition& kernel = kit->second;
                const XElement& groups = One(*ins, "Groups");
                Check(groups, "Groups", {"x", "y", "z"}, {});
                launch.groups[0] = static_cast<uint32_t>(Integer(groups, "x", true));
                launch.groups[1] = static_cast<uint32_t>(Integer(groups, "y", true));
                launch.groups[2] = static_cast<uint32_t>(Integer(groups, "z", true));
                launch.threads = kernel.threads;
                for (const auto& a : ReadArguments(*ins)) {
                    const auto kp = kernel.parameters.find(a.parameter);
                    if (kp == kernel.parameters.end())
                        Bad("Dispatch binds an unknown kernel parameter '" + a.parameter + "'.");
                    Bound b = orchestration_argument(a.source);
                    if (kp->second.access == VmAccess::ReadWrite && b.access != VmAccess::ReadWrite)
                        Bad("Dispatch binds writable kernel parameter '" + a.parameter + "' to a read-only one.");
                    b.tensor = kp->second.tensor;
                    b.access = kp->second.access;
                    b.offset += a.offset;
                    if (!kernel_bound.emplace(a.parameter, b).second)
                        Bad("Dispatch binds '" + a.parameter + "' twice.");
                }
                if (kernel_bound.size() != kernel.parameters.size())
                    Bad("Dispatch of '" + launch.definition + "' leaves kernel parameters unbound.");
                const auto& knodes = kernel.nodes->children;
                if (knodes.size() != 1)
                    throw NotSupportedException("Kernel definition '" + launch.definition +
                                                "': the HIP executor runs kernels of one operator.");
                Check(knodes[0], "Node", {"id"}, {"Dependencies", "Operator"});
                op = &One(knodes[0], "Operator");
                resolve = [&](const std::string& name) -> Bound {
                    const auto it = kernel_bound.find(name);
                    if (it == kernel_bound.end())
                        Bad("Operator argument names an unbound kernel parameter '" + name + "'.");
                    return it->second;
                };
            } else if (ins->name != "Operator") {
                throw NotSupportedException("Entry '" + entry + "': " + ins->name +
                                            " nodes have no HIP execution (operators and dispatches only).");
            }
            Check(*op, "Operator", {"name", "collection"},
                  {"Arguments", "Precision", "ResolvedPrecision", "ExecutionConfiguration", "Attributes", "IndexBounds",
                   "ParameterAccesses"});
            const XElement& prec = One(*op, "Precision");
            Check(prec, "Precision", {"minimumArithmeticType", "minimumAccumulatorType"}, {});
            const PrecisionRequirement requirement{
                EnumValue<GraphElementType>(prec, "minimumArithmeticType", kElementTypes),
                EnumValue<GraphElementType>(prec, "minimumAccumulatorType", kElementTypes)};
            if (const XElement* rp = OptionalOne(*op, "ResolvedPrecision")) {
                Check(*rp, "ResolvedPrecision", {"arithmeticType", "accumulatorType"}, {});
                EnumValue<GraphElementType>(*rp, "arithmeticType", kElementTypes);
                EnumValue<GraphElementType>(*rp, "accumulatorType", kElementTypes);
            }
            if (const XElement* ec = OptionalOne(*op, "ExecutionConfiguration")) {
                Check(*ec, "ExecutionConfiguration", {"target", "implementation"}, {});
                if (Required(*ec, "target") != kExecutionTarget)
                    Bad("Unknown execution configuration target.");
                const std::string& impl = Required(*ec, "implementation");
                const std::string variant = ".any_shape";
                if (impl.size() > variant.size() && impl.compare(impl.size() - variant.size(), variant.size(), variant) == 0)
                    launch.implementation_variant = "any_shape";
            }
            std::vector<InstructionParameter> params;
            std::set<std::string> names;
            if (const XElement* attrs = OptionalOne(*op, "Attributes")) {
                Check(*attrs, "Attributes", {}, {"Attribute"});
                for (const auto& a : attrs->children) {
                    Check(a, "Attribute", {"name", "value"}, {});
                    if (!names.insert(Required(a, "name")).second)
                        Bad("Duplicate operator attribute.");
                    params.push_back(InstructionParameter::Attribute(Required(a, "name"), Required(a, "value")));
                }
            }
            if (const XElement* bounds = OptionalOne(*op, "IndexBounds")) {
                Check(*bounds, "IndexBounds", {}, {"Bound"});
                if (!bounds->children.empty())
                    throw NotSupportedException("Index bounds have no HIP execution.");
            }
            std::map<std::string, GraphResourceAccess> accesses;
            if (const XElement* ports = OptionalOne(*op, "ParameterAccesses")) {
                Check(*ports, "ParameterAccesses", {}, {"Port"});
                for (const auto& port : ports->children) {
                    Check(port, "Port", {"name", "access"}, {});
                    if (!accesses.emplace(Required(port, "name"),
                                          EnumValue<GraphResourceAccess>(port, "access", kResourceAccess))
                             .second)
                        Bad("Duplicate port access.");
                }
            }
            const auto instruction = registry->Resolve(Required(*op, "collection"), Required(*op, "name"),
                                                       InstructionTarget::Hip());
            for (const auto& a : ReadArguments(*op)) {
                const Bound b = resolve(a.source);
                if (!names.insert(a.parameter).second)
                    Bad("Duplicate operator argument '" + a.parameter + "'.");
                const auto acc = accesses.find(a.parameter);
                const GraphResourceAccess access = acc != accesses.end()              ? acc->second
                                                   : b.access == VmAccess::ReadWrite ? GraphResourceAccess::ReadWrite
                                                                                     : GraphResourceAccess::Read;
                if (access != GraphResourceAccess::Read && b.access != VmAccess::ReadWrite)
                    Bad("Operator argument '" + a.parameter + "' writes read-only parameter '" + a.source + "'.");
                params.push_back(InstructionParameter::Tensor(a.parameter, b.tensor, access, b.slot, b.offset + a.offset));
            }
            if (launch.definition.empty() && launch.implementation_variant.empty())
                p.AddDispatch(entry, instruction, params, requirement);
            else
                p.AddKernelDispatch(entry, instruction, params, requirement, launch);
        }
    }
    return p;
}

// ---- SHA-256 (FIPS 180-4) ------------------------------------------------------------------

std::string Sha256Hex(const void* data, size_t length)
{
    static const uint32_t K[64] = {
        0x428a2f98, 0x71374491, 0xb5c0fbcf, 0xe9b5dba5, 0x3956c25b, 0x59f111f1, 0x923f82a4, 0xab1c5ed5,
        0xd807aa98, 0x12835b01, 0x243185be, 0x550c7dc3, 0x72be5d74, 0x80deb1fe, 0x9bdc06a7, 0xc19bf174,
        0xe49b69c1, 0xefbe4786, 0x0fc19dc6, 0x240ca1cc, 0x2de92c6f, 0x4a7484aa, 0x5cb0a9dc, 0x76f988da,
        0x983e5152, 0xa831c66d, 0xb00327c8, 0xbf597fc7, 0xc6e00bf3, 0xd5a79147, 0x06ca6351, 0x14292967,
        0x27b70a85, 0x2e1b2138, 0x4d2c6dfc, 0x53380d13, 0x650a7354, 0x766a0abb, 0x81c2c92e, 0x92722c85,
        0xa2bfe8a1, 0xa81a664b, 0xc24b8b70, 0xc76c51a3, 0xd192e819, 0xd6990624, 0xf40e3585, 0x106aa070,
        0x19a4c116, 0x1e376c08, 0x2748774c, 0x34b0bcb5, 0x391c0cb3, 0x4ed8aa4a, 0x5b9cca4f, 0x682e6ff3,
        0x748f82ee, 0x78a5636f, 0x84c87814, 0x8cc70208, 0x90befffa, 0xa4506ceb, 0xbef9a3f7, 0xc67178f2};
    uint32_t h[8] = {0x6a09e667, 0xbb67ae85, 0x3c6ef372, 0xa54ff53a, 0x510e527f, 0x9b05688c, 0x1f83d9ab, 0x5be0cd19};
    const auto rotr = [](uint32_t x, int n) { return (x >> n) | (x << (32 - n)); };
    std::vector<uint8_t> m(static_cast<const uint8_t*>(data), static_cast<const uint8_t*>(data) + length);
    const uint64_t bits = static_cast<uint64_t>(length) * 8;
    m.push_back(0x80);
    while (m.size() % 64 != 56)
        m.push_back(0);
    for (int i = 7; i >= 0; i--)
        m.push_back(static_cast<uint8_t>(bits >> (8 * i)));
    for (size_t off = 0; off < m.size(); off += 64) {
        uint32_t w[64];
        for (int i = 0; i < 16; i++)
            w[i] = (static_cast<uint32_t>(m[off + 4 * i]) << 24) | (static_cast<uint32_t>(m[off + 4 * i + 1]) << 16) |
                   (static_cast<uint32_t>(m[off + 4 * i + 2]) << 8) | m[off + 4 * i + 3];
        for (int i = 16; i < 64; i++) {
            const uint32_t s0 = rotr(w[i - 15], 7) ^ rotr(w[i - 15], 18) ^ (w[i - 15] >> 3);
            const uint32_t s1 = rotr(w[i - 2], 17) ^ rotr(w[i - 2], 19) ^ (w[i - 2] >> 10);
            w[i] = w[i - 16] + s0 + w[i - 7] + s1;
        }
        uint32_t a = h[0], b = h[1], c = h[2], d = h[3], e = h[4], f = h[5], g = h[6], hh = h[7];
        for (int i = 0; i < 64; i++) {
            const uint32_t S1 = rotr(e, 6) ^ rotr(e, 11) ^ rotr(e, 25);
            const uint32_t ch = (e & f) ^ (~e & g);
            const uint32_t t1 = hh + S1 + ch + K[i] + w[i];
            const uint32_t S0 = rotr(a, 2) ^ rotr(a, 13) ^ rotr(a, 22);
            const uint32_t maj = (a & b) ^ (a & c) ^ (b & c);
            const uint32_t t2 = S0 + maj;
            hh = g;
            g = f;
            f = e;
            e = d + t1;
            d = c;
            c = b;
            b = a;
            a = t1 + t2;
        }
        h[0] += a; h[1] += b; h[2] += c; h[3] += d; h[4] += e; h[5] += f; h[6] += g; h[7] += hh;
    }
    static const char* hex = "0123456789ABCDEF";
    std::string out;
    for (const uint32_t v : h)
        for (int i = 28; i >= 0; i -= 4)
            out += hex[(v >> i) & 15];
    return out;
}

namespace {

// ---- stored ZIP (APPNOTE 6.3: local headers, central directory, end record) ----------------

uint32_t Crc32(const uint8_t* p, size_t n)
{
    uint32_t c = 0xFFFFFFFFu;
    for (size_t i = 0; i < n; i++) {
        c ^= p[i];
        for (int k = 0; k < 8; k++)
            c = (c >> 1) ^ (0xEDB88320u & (0u - (c & 1u)));
    }
    return ~c;
}

void Put16(std::vector<uint8_t>& b, uint32_t v)
{
    b.push_back(static_cast<uint8_t>(v));
    b.push_back(static_cast<uint8_t>(v >> 8));
}
void Put32(std::vector<uint8_t>& b, uint32_t v)
{
    Put16(b, v & 0xFFFF);
    Put16(b, v >> 16);
}
uint32_t Get16(const std::vector<uint8_t>& b, size_t i) { return b[i] | (static_cast<uint32_t>(b[i + 1]) << 8); }
uint32_t Get32(const std::vector<uint8_t>& b, size_t i) { return Get16(b, i) | (Get16(b, i + 2) << 16); }

std::vector<uint8_t> WriteZip(const std::vector<std::pair<std::string, std::string>>& files)
{
    std::vector<uint8_t> out, central;
    for (const auto& [name, data] : files) {
        const uint32_t crc = Crc32(reinterpret_cast<const uint8_t*>(data.data()), data.size());
        const uint32_t offset = static_cast<uint32_t>(out.size());
        Put32(out, 0x04034b50);
        Put16(out, 20); Put16(out, 0x0800); Put16(out, 0);   // version, UTF-8 names, stored
        Put16(out, 0); Put16(out, 0x21);                     // time, date (1980-01-01)
        Put32(out, crc); Put32(out, static_cast<uint32_t>(data.size())); Put32(out, static_cast<uint32_t>(data.size()));
        Put16(out, static_cast<uint32_t>(name.size())); Put16(out, 0);
        out.insert(out.end(), name.begin(), name.end());
        out.insert(out.end(), data.begin(), data.end());
        Put32(central, 0x02014b50);
        Put16(central, 20); Put16(central, 20); Put16(central, 0x0800); Put16(central, 0);
        Put16(central, 0); Put16(central, 0x21);
        Put32(central, crc); Put32(central, static_cast<uint32_t>(data.size()));
        Put32(central, static_cast<uint32_t>(data.size()));
        Put16(central, static_cast<uint32_t>(name.size())); Put16(central, 0); Put16(central, 0);
        Put16(central, 0); Put16(central, 0); Put32(central, 0); Put32(central, offset);
        central.insert(central.end(), name.begin(), name.end());
    }
    const uint32_t cd_offset = static_cast<uint32_t>(out.size());
    out.insert(out.end(), central.begin(), central.end());
    Put32(out, 0x06054b50);
    Put16(out, 0); Put16(out, 0);
    Put16(out, static_cast<uint32_t>(files.size())); Put16(out, static_cast<uint32_t>(files.size()));
    Put32(out, static_cast<uint32_t>(central.size())); Put32(out, cd_offset);
    Put16(out, 0);
    return out;
}

// Reads a stored ZIP through its central directory, with the reference's
// limits (D3D12VmArtifact.cs:120-124): at most 10000 entries, 64 MiB each,
// 512 MiB in all, unique names; CRC-32 checked.
std::map<std::string, std::string> ReadZip(const std::vector<uint8_t>& b)
{
    const auto bad = [] { Bad("Invalid or oversized HIP VM archive."); };
    if (b.size() < 22)
        bad();
    size_t eocd = std::string::npos;
    for (size_t i = b.size() - 22 + 1; i-- > 0 && b.size() - i <= 22 + 65535;)
        if (Get32(b, i) == 0x06054b50) {
            eocd = i;
            break;
        }
    if (eocd == std::string::npos)
        bad();
    const uint32_t count = Get16(b, eocd + 10), cd_size = Get32(b, eocd + 12), cd_off = Get32(b, eocd + 16);
    if (count > 10000 || static_cast<uint64_t>(cd_off) + cd_size > eocd)
        bad();
    std::map<std::string, std::string> files;
    uint64_t total = 0;
    size_t p = cd_off;
    for (uint32_t k = 0; k < count; k++) {
        if (p + 46 > eocd || Get32(b, p) != 0x02014b50)
            bad();
        const uint32_t method = Get16(b, p + 10), crc = Get32(b, p + 16), csize = Get32(b, p + 20),
                       usize = Get32(b, p + 24), nlen = Get16(b, p + 28), xlen = Get16(b, p + 30),
                       clen = Get16(b, p + 32), lho = Get32(b, p + 42);
        if (method != 0 || csize != usize || usize > 64u * 1024 * 1024 || p + 46 + nlen + xlen + clen > eocd)
            bad();
        const std::string name(reinterpret_cast<const char*>(&b[p + 46]), nlen);
        p += 46 + nlen + xlen + clen;
        if (static_cast<uint64_t>(lho) + 30 > b.size() || Get32(b, lho) != 0x04034b50)
            bad();
        const uint64_t data = static_cast<uint64_t>(lho) + 30 + Get16(b, lho + 26) + Get16(b, lho + 28);
        if (data + usize > cd_off)
            bad();
        total += usize;
        if (total > 512ull * 1024 * 1024)
            bad();
        if (Crc32(&b[data], usize) != crc)
            Bad("Artifact integrity check failed.");
        if (!files.emplace(name, std::string(reinterpret_cast<const char*>(&b[data]), usize)).second)
            bad();
    }
    return files;
}

// ---- the manifest's JSON: one flat object of string and integer members --------------------

std::map<std::string, std::string> JsonObject(const std::string& s)
{
    const auto bad = [] { Bad("Invalid artifact manifest."); };
    size_t i = 0;
    const auto skip = [&] {
        while (i < s.size() && (s[i] == ' ' || s[i] == '\n' || s[i] == '\r' || s[i] == '\t'))
            i++;
    };
    const auto str = [&] {
        if (i >= s.size() || s[i] != '"')
            bad();
        std::string v;
        for (i++; i < s.size() && s[i] != '"'; i++) {
            if (s[i] != '\\') {
                v += s[i];
                continue;
            }
            if (++i >= s.size())
                bad();
            switch (s[i]) {
            case '"': v += '"'; break;
            case '\\': v += '\\'; break;
            case '/': v += '/'; break;
            case 'n': v += '\n'; break;
            case 'r': v += '\r'; break;
            case 't': v += '\t'; break;
            case 'b': v += '\b'; break;
            case 'f': v += '\f'; break;
            case 'u': {
                if (i + 4 >= s.size())
                    bad();
                const unsigned long c = std::stoul(s.substr(i + 1, 4), nullptr, 16);
                if (c >= 0x80)
                    bad();   // the manifest's strings are ASCII
                v += static_cast<char>(c);
                i += 4;
                break;
            }
            default: bad();
            }
        }
        if (i >= s.size())
            bad();
        i++;
        return v;
    };
    std::map<std::string, std::string> out;
    skip();
    if (i >= s.size() || s[i] != '{')
        bad();
    i++;
    skip();
    if (i < s.size() && s[i] == '}') {
        i++;
    } else {
        for (;;) {
            skip();
            const std::string key = str();
            skip();
            if (i >= s.size() || s[i] != ':')
                bad();
            i++;
            skip();
            std::string value;
            if (i < s.size() && s[i] == '"') {
                value = str();
            } else {
                const size_t b = i;
                while (i < s.size() && (std::isdigit(static_cast<unsigned char>(s[i])) || s[i] == '-'))
                    i++;
                if (i == b)
                    bad();
                value = s.substr(b, i - b);
            }
            if (!out.emplace(key, value).second)
                bad();
            skip();
            if (i < s.size() && s[i] == ',') {
                i++;
                continue;
            }
            if (i < s.size() && s[i] == '}') {
                i++;
                break;
            }
            bad();
        }
    }
    skip();
    if (i != s.size())
        bad();
    return out;
}

constexpr int kArtifactVersion = 1;

}  // namespace

std::vector<uint8_t> ExportHipVmArtifact(const HipVmProgram& program)
{
    const std::string xml = SerializeVmProgram(program);
    const std::string manifest = "{\"Version\":" + std::to_string(kArtifactVersion) +
                                 ",\"BackendAbi\":" + JsonString(HipVmArtifactAbi) + ",\"Target\":" +
                                 JsonString(kExecutionTarget) + ",\"LibraryAbi\":" + std::to_string(si_hip_abi_version()) +
                                 ",\"ProgramHash\":" + JsonString(Sha256Hex(xml.data(), xml.size())) + "}";
    const std::string envelope = "{\"Manifest\":" + JsonString(manifest) + ",\"Sha256\":" +
                                 JsonString(Sha256Hex(manifest.data(), manifest.size())) + "}";
    return WriteZip({{"program.xml", xml}, {"manifest.json", envelope}});
}

HipVmProgram ImportHipVmArtifact(const std::vector<uint8_t>& archive,
                                 const std::shared_ptr<const InstructionRegistry>& registry)
{
    const auto files = ReadZip(archive);
    const auto get = [&](const char* name) -> const std::string& {
        const auto it = files.find(name);
        if (it == files.end())
            Bad(std::string("Artifact entry '") + name + "' is missing.");
        return it->second;
    };
    const auto envelope = JsonObject(get("manifest.json"));
    if (envelope.size() != 2 || !envelope.count("Manifest") || !envelope.count("Sha256"))
        Bad("Missing artifact manifest.");
    const std::string& manifest_text = envelope.at("Manifest");
    if (envelope.at("Sha256") != Sha256Hex(manifest_text.data(), manifest_text.size()))
        Bad("Manifest integrity check failed.");
    const auto manifest = JsonObject(manifest_text);
    const auto field = [&](const char* k) -> const std::string& {
        const auto it = manifest.find(k);
        if (it == manifest.end())
            Bad("Invalid artifact manifest.");
        return it->second;
    };
    if (field("Version") != std::to_string(kArtifactVersion) || field("BackendAbi") != HipVmArtifactAbi ||
        field("Target") != kExecutionTarget)
        Bad("Unsupported HIP VM artifact target/version/ABI.");
    if (field("LibraryAbi") != std::to_string(si_hip_abi_version()))
        Bad("The artifact was exported against another libsharpinference_hip ABI.");
    const std::string& xml = get("program.xml");
    if (field("ProgramHash") != Sha256Hex(xml.data(), xml.size()))
        Bad("Artifact integrity check failed.");
    if (files.size() != 2)
        Bad("Unexpected artifact entries.");
    return DeserializeVmProgram(xml, registry);
}

}  // namespace sharpinference
